"""KittyPagedAttention — drop-in attention module over the Kitty KV cache.

Same constructor and ``forward(q, k, v, seq_id=0, attention_mask=None)`` as
the reference (``kitty/attention.py:28-191``), plus batching: the reference
asserts B == 1 (``:100``); here row b of a (B, ...) call belongs to sequence
``seq_id[b]`` (a sequence of ids) or ``seq_id + b`` (an int).

Decode (T == 1): the new K/V of all B sequences go through the pipeline (one
append launch, and a batch-quantize launch for the sequences whose key or
value buffer fills), then one fused split-K paged decode attends sinks,
pages and the FP16 key / value tails of every sequence at once.  The decode
plan of a batch (its validated kernel arguments and workspace) is built once
per (layer, slot range) and reused while a batch occupies the same
contiguous range of pipeline slots: it reads lengths, block table and
buffers from the pipeline's device state, so a step only rebinds q and the
output.  No step waits for the GPU.

Prefill (T > 1): the chunk goes into the pipeline in bulk (sinks and buffer
rows copied, every complete page quantised straight from the chunk in one
launch per sequence; the same state as pushing the tokens one at a time,
which is what the reference does, ``:169-177``), and the output is causal
attention over the chunk, as the reference computes it (``:179-191``); it
runs in float32 (torch's SDPA math path).

Pools and buffers on the CPU (``KittyConfig.device = "cpu"``, the reference's
config-1 plumbing case) run the same steps with the torch code of
``kernels.cpu``; device pools only ever run the HIP kernels.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from .config import KittyConfig
from .layout import PageCentricKVLayoutManager
from .pipeline import KittyInferencePipeline
from .kernels.ops import DecodePlan, boost_rows_unique, decode_plan


class KittyPagedAttention(nn.Module):
    def __init__(self, config: KittyConfig, num_q_heads: int, layout: PageCentricKVLayoutManager,
                 pipeline: KittyInferencePipeline, layer_id: int) -> None:
        super().__init__()
        self.config = config
        self.num_q_heads = num_q_heads
        self.num_kv_heads = config.num_kv_heads
        self.head_dim = config.head_dim
        self.q_per_kv = num_q_heads // config.num_kv_heads
        self.layer_id = layer_id
        self.layout = layout
        self.pipeline = pipeline
        self.scale = 1.0 / math.sqrt(config.head_dim)
        self._boost_unique = boost_rows_unique(pipeline.boost_idx_uint8[layer_id], config.d_boost)
        self._plans: dict = {}   # tuple(slots) -> DecodePlan over the pipeline's device state

    def _seq_ids(self, B: int, seq_id: Union[int, Sequence[int]]) -> List[int]:
        if isinstance(seq_id, int):
            return [seq_id + b for b in range(B)]
        ids = [int(s) for s in seq_id]
        if len(ids) != B:
            raise ValueError(f"{len(ids)} sequence ids for a batch of {B}")
        return ids

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                seq_id: Union[int, Sequence[int]] = 0, attention_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, nqh, T, D = q.shape
        assert nqh == self.num_q_heads
        assert D == self.head_dim
        seq_ids = self._seq_ids(B, seq_id)
        if T == 1:
            return self._decode_step(q, k, v, seq_ids)
        return self._prefill(q, k, v, seq_ids)

    def _plan(self, qd: torch.Tensor, seq_ids: List[int]) -> DecodePlan:
        key = tuple(self.pipeline.slot(s) for s in seq_ids)
        plan = self._plans.get(key)
        if plan is not None:
            return plan
        x = self.pipeline.decode_inputs(self.layer_id, seq_ids, full_width=True)
        lay = self.layout
        plan = decode_plan(qd, x["block_table"], x["num_pages"], lay.key_baseline, lay.key_boost, lay.key_metadata,
                          lay.value_pool, lay.value_metadata, self.pipeline.boost_idx_uint8[self.layer_id],
                          x["sink_k"], x["sink_v"], x["sink_len"], x["tail_k"], x["tail_v"], x["tail_len"],
                          max_pages=x["max_pages"], sm_scale=self.scale, boost_unique=self._boost_unique,
                          num_pages_v=x["num_pages_v"], tail_len_v=x["tail_len_v"])
        if x["contiguous"]:      # views of the pipeline's state: valid for every later step
            if len(self._plans) >= 16:
                self._plans.clear()
            self._plans[key] = plan
        return plan

    def _decode_step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seq_ids: List[int]) -> torch.Tensor:
        self.pipeline.push_tokens(self.layer_id, k[:, :, 0], v[:, :, 0], seq_ids)
        qd = q[:, :, 0].to(self.pipeline.buffer_dtype).contiguous()
        plan = self._plan(qd, seq_ids)
        out = torch.empty(qd.shape, dtype=torch.float16, device=qd.device)
        return plan.run_with(qd, out).unsqueeze(2).to(q.dtype)

    def _prefill(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seq_ids: List[int]) -> torch.Tensor:
        self.pipeline.push_chunk(self.layer_id, k, v, seq_ids)
        k_exp = k.float().repeat_interleave(self.q_per_kv, dim=1)
        v_exp = v.float().repeat_interleave(self.q_per_kv, dim=1)
        out = F.scaled_dot_product_attention(q.float(), k_exp, v_exp, attn_mask=None, dropout_p=0.0,
                                             is_causal=True, scale=self.scale)
        return out.to(q.dtype)


class KittyAttentionFactory:
    """Builds the layout, the pipeline and one module per layer (attention.py:198-257)."""

    @classmethod
    def from_config(cls, config: KittyConfig, boost_idx_uint8: torch.Tensor,
                    num_q_heads: int) -> Tuple[PageCentricKVLayoutManager, KittyInferencePipeline,
                                               List[KittyPagedAttention]]:
        layout = PageCentricKVLayoutManager(config, boost_idx_uint8)
        pipeline = KittyInferencePipeline(config, layout, boost_idx_uint8)
        layers = [KittyPagedAttention(config, num_q_heads, layout, pipeline, i) for i in range(config.num_layers)]
        return layout, pipeline, layers
