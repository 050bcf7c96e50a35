"""Channel-sensitivity profiler: which key channels get INT4.

Drop-in for ``KittySensitivityProfiler`` (reference ``kitty/sensitivity.py:75-330``):
same constructor, hook registration on the key projections, ``compute``,
``save`` / ``load`` and the ``boost_masks`` / ``boost_idx_uint8``
properties, and the same on-disk files, so profiles are interchangeable
with the reference:

    scores.pt       float32 (L, H, D)  mean |k| per (layer, KV head, channel)
    boost_masks.pt  bool    (L, H, D)  True for the d_boost top channels
    boost_idx.pt    uint8   (L, H, D)  rank 0..d_boost-1 of a boosted channel, else the sentinel
    meta.json       config snapshot and calibration token counts per layer

The per-(head, channel) sum of |k| is accumulated on the ROCm device by
``kitty_channel_abs_sum`` (fixed summation order); keys on the CPU are summed
with torch there.  Ranks come from a stable
descending sort, so equal scores rank by channel index; the reference's
``argsort`` leaves the order of ties unspecified.
"""
from __future__ import annotations

import ctypes
import json
from pathlib import Path
from typing import Callable, Dict, List, Optional, Sequence

import torch
import torch.nn as nn

from . import _hip
from .config import KittyConfig


class _ChannelAccumulator:
    """Running sum of |k| per (KV head, channel) of one layer (sensitivity.py:34-67)."""

    def __init__(self, num_kv_heads: int, head_dim: int, device) -> None:
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self._sum_abs = torch.zeros(num_kv_heads, head_dim, dtype=torch.float32, device=device)
        self.token_count = 0
        # per-chunk running sums of the deferred kernel (zero between flushes),
        # added into _sum_abs when sum_abs is read: one pass over the keys per
        # update, the finishing pass once per read
        self._slots: Optional[torch.Tensor] = None
        self._pending = False

    @property
    def sum_abs(self) -> torch.Tensor:
        """Σ|k| per (head, channel) over every update so far (fp32 (H, D))."""
        if self._pending:
            _hip.check(_hip.load().kitty_channel_abs_sum_flush(
                self._slots.data_ptr(), self.num_kv_heads, self.head_dim, self._sum_abs.data_ptr(),
                _hip.stream_ptr(self._sum_abs.device)))
            self._pending = False
        return self._sum_abs

    @torch.no_grad()
    def update(self, key: torch.Tensor) -> None:
        """key (batch, num_kv_heads, seq_len, head_dim) fp16 / bf16 on the ROCm
        device (a CPU key is summed with torch on the CPU)."""
        B, H, T, D = key.shape
        if (H, D) != (self.num_kv_heads, self.head_dim):
            raise ValueError(f"key shape {tuple(key.shape)} does not match ({self.num_kv_heads}, {self.head_dim})")
        if key.device.type == "cpu":
            self._sum_abs = self.sum_abs.cpu() + key.abs().float().sum(dim=(0, 2))
            self.token_count += B * T
            return
        dev = _hip.require_device(key)
        if self._sum_abs.device != dev:
            self._sum_abs = self.sum_abs.to(dev)      # pending slots flushed on the old device first
            self._slots = None
        if key.dtype not in (torch.float16, torch.bfloat16):
            key = key.to(torch.float16)  # the kernel reads fp16 or bf16 (a model's dtype)
        if key.stride(3) != 1:
            key = key.contiguous()
        L = _hip.load()
        if self._slots is None:
            need = ctypes.c_size_t(0)
            _hip.check(L.kitty_channel_abs_sum_deferred_size(H, D, ctypes.byref(need)))
            self._slots = torch.zeros(max(need.value, 16), dtype=torch.uint8, device=dev)
            self._slots_bytes = need.value
        _hip.check(L.kitty_channel_abs_sum_deferred(
            key.data_ptr(), key.stride(0), key.stride(2), key.stride(1), B, T, H, D, _hip.dtype_code(key, "key"),
            self._sum_abs.data_ptr(), self._slots.data_ptr() if self._slots_bytes else None, self._slots_bytes,
            _hip.stream_ptr(dev)))
        self._pending = self._slots_bytes > 0
        self.token_count += B * T

    def scores(self) -> torch.Tensor:
        if self.token_count == 0:
            raise RuntimeError("No tokens have been accumulated yet.")
        return self.sum_abs / self.token_count


def rank_channels(scores: torch.Tensor, d_boost: int, sentinel: int):
    """scores (L, H, D) -> (boost_masks bool, boost_idx uint8): the d_boost
    channels of highest score per (layer, head) get ranks 0.. in descending
    score order (sensitivity.py:191-203); ties rank by channel index."""
    scores = scores.detach().float().cpu()
    order = torch.argsort(scores, dim=-1, descending=True, stable=True)
    boost_idx = torch.full(scores.shape, sentinel, dtype=torch.uint8)
    boost_idx.scatter_(-1, order[..., :d_boost], torch.arange(d_boost, dtype=torch.uint8).expand(
        *scores.shape[:-1], d_boost).contiguous())
    masks = boost_idx < d_boost if d_boost > 0 else torch.zeros(scores.shape, dtype=torch.bool)
    return masks, boost_idx


class KittySensitivityProfiler:
    """Offline profiler: hook the key projections, run calibration data,
    rank channels by mean |k| and keep the top d_boost of each (layer, head)
    for INT4 (sensitivity.py:75-330)."""

    def __init__(self, config: KittyConfig, model: Optional[nn.Module] = None) -> None:
        self.config = config
        self.model = model
        self._accumulators: Dict[int, _ChannelAccumulator] = {}
        self._hooks: List[torch.utils.hooks.RemovableHandle] = []
        self.scores_: Optional[torch.Tensor] = None
        self.boost_masks_: Optional[torch.Tensor] = None
        self.boost_idx_uint8_: Optional[torch.Tensor] = None

    # ------------------------------------------------------------------ hooks
    def accumulator(self, layer_idx: int) -> _ChannelAccumulator:
        acc = self._accumulators.get(layer_idx)
        if acc is None:
            acc = _ChannelAccumulator(self.config.num_kv_heads, self.config.head_dim, self.config.device)
            self._accumulators[layer_idx] = acc
        return acc

    def update(self, layer_idx: int, key: torch.Tensor) -> None:
        """Feed keys (B, H, T, D) of one layer directly, without hooks."""
        self.accumulator(layer_idx).update(key)

    def register_hooks(self, layer_indices: Sequence[int],
                       key_proj_getter: Optional[Callable[[nn.Module, int], nn.Module]] = None) -> None:
        """Forward hooks on the key projections (sensitivity.py:108-160): the
        projection output (B, T, H*D) is viewed as (B, H, T, D) keys."""
        if self.model is None:
            raise RuntimeError("A model must be provided to KittySensitivityProfiler to register hooks.  "
                               "Pass model= at construction time.")
        for layer_idx in layer_indices:
            acc = self.accumulator(layer_idx)
            k_proj = self._find_key_proj(layer_idx, key_proj_getter)

            def hook(module, inp, out, acc=acc):
                B, T, _ = out.shape
                acc.update(out.detach().reshape(B, T, acc.num_kv_heads, acc.head_dim).permute(0, 2, 1, 3))

            self._hooks.append(k_proj.register_forward_hook(hook))

    def remove_hooks(self) -> None:
        for h in self._hooks:
            h.remove()
        self._hooks.clear()

    def _find_key_proj(self, layer_idx: int, getter: Optional[Callable[[nn.Module, int], nn.Module]]) -> nn.Module:
        """The key projection of a layer: `getter` or the usual attribute paths
        (sensitivity.py:283-330)."""
        if getter is not None:
            return getter(self.model, layer_idx)
        candidates = [
            lambda m, i: m.layers[i].self_attn.k_proj,
            lambda m, i: m.model.layers[i].self_attn.k_proj,
            lambda m, i: m.transformer.h[i].attn.k_proj,
        ]
        for fn in candidates:
            try:
                return fn(self.model, layer_idx)
            except (AttributeError, IndexError, TypeError):
                continue
        raise AttributeError(f"no key projection found for layer {layer_idx}; pass key_proj_getter=")

    # ----------------------------------------------------------------- compute
    def compute(self) -> None:
        """Scores, masks and boost indices from the accumulated sums (sensitivity.py:164-207)."""
        cfg = self.config
        if not self._accumulators:
            raise RuntimeError("No accumulators found.  Did you call register_hooks() and "
                               "forward the model over the calibration data?")
        scores = torch.zeros(cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, dtype=torch.float32)
        for layer_idx, acc in self._accumulators.items():
            scores[layer_idx] = acc.scores().cpu()
        self.scores_ = scores
        self.boost_masks_, self.boost_idx_uint8_ = rank_channels(scores, cfg.d_boost, cfg.sentinel)

    # ------------------------------------------------------------------- I/O
    def save(self, directory) -> None:
        """scores.pt, boost_masks.pt, boost_idx.pt, meta.json (sensitivity.py:211-245)."""
        if self.scores_ is None:
            self.compute()
        directory = Path(directory)
        directory.mkdir(parents=True, exist_ok=True)
        torch.save(self.scores_, directory / "scores.pt")
        torch.save(self.boost_masks_, directory / "boost_masks.pt")
        torch.save(self.boost_idx_uint8_, directory / "boost_idx.pt")
        meta = {
            "num_layers": self.config.num_layers,
            "num_kv_heads": self.config.num_kv_heads,
            "head_dim": self.config.head_dim,
            "d_boost": self.config.d_boost,
            "boost_rate": self.config.boost_rate,
            "token_count": {k: v.token_count for k, v in self._accumulators.items()},
        }
        with open(directory / "meta.json", "w") as f:
            json.dump(meta, f, indent=2)

    @classmethod
    def load(cls, directory, config: KittyConfig) -> "KittySensitivityProfiler":
        """Read a saved profile (ours or the reference's): tensors only, no pickled code."""
        directory = Path(directory)
        prof = cls(config)
        prof.scores_ = torch.load(directory / "scores.pt", weights_only=True)
        prof.boost_masks_ = torch.load(directory / "boost_masks.pt", weights_only=True)
        prof.boost_idx_uint8_ = torch.load(directory / "boost_idx.pt", weights_only=True)
        return prof

    def summary(self) -> str:
        """Human-readable summary with the reference's lines (sensitivity.py:313-332):
        shape, boost rate and INT4 channels per head, sentinel, and the
        largest and mean channel score once computed."""
        cfg = self.config
        if self.scores_ is None:
            return "KittySensitivityProfiler — not yet computed."
        return "\n".join([
            "KittySensitivityProfiler Summary",
            f"  Layers: {cfg.num_layers}, KV Heads: {cfg.num_kv_heads}, Head Dim: {cfg.head_dim}",
            f"  Boost rate: {cfg.boost_rate:.1%} → {cfg.d_boost} INT4 channels/head",
            f"  Sentinel value: {cfg.sentinel}",
            f"  Max channel score: {self.scores_.max().item():.4f}",
            f"  Mean channel score: {self.scores_.mean().item():.4f}",
        ])

    @property
    def boost_masks(self) -> torch.Tensor:
        if self.boost_masks_ is None:
            self.compute()
        return self.boost_masks_

    @property
    def boost_idx_uint8(self) -> torch.Tensor:
        if self.boost_idx_uint8_ is None:
            self.compute()
        return self.boost_idx_uint8_
