"""Token state machine of the Kitty KV cache, device-resident and batched.

Drop-in for ``KittyInferencePipeline`` (reference ``kitty/pipeline.py:49-326``):
same constructor, ``push_token``, ``get_attention_context``,
``reset_sequence``, ``stats`` and counter attributes.  Differences, all
deliberate:

* Every sequence gets its own slot of FP16 buffers and every (slot, layer) its
  own counters.  The reference keeps one shared set and advances counters only
  on layer 0 (``pipeline.py:90-111, 146-177``), so layers >= 1 and a second
  sequence overwrite each other.
* A spill quantises the G buffered tokens of key AND value into the same page,
  so page p holds K and V of the same tokens and the FP16 key and value tails
  have equal length (the contract of ``paged_attention_reference``,
  ``kernels/attention.py:163-165``).  The reference quantises the values
  evicted from its R-window instead, which pairs keys of page p with values of
  page p-1 and zeros in page 0.  ``val_local_len`` therefore reports the
  length of the FP16 value tail (equal to ``key_qbuf_len``) and
  ``val_qbuf_len`` is always 0.
* A spill is one launch of the batch quantize kernel for every sequence that
  filled its buffer in that step.

Host state is a few integer arrays; nothing here synchronises with the GPU
except reading the physical page ids the allocator hands out.
"""
from __future__ import annotations

from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import numpy as np
import torch

from .config import KittyConfig
from .layout import PageCentricKVLayoutManager
from .kernels.ops import pool_store, quantize_into_pools


class KittyInferencePipeline:
    def __init__(self, config: KittyConfig, layout: PageCentricKVLayoutManager, boost_idx_uint8: torch.Tensor,
                 num_slots: Optional[int] = None) -> None:
        if config.dtype != "float16":
            raise NotImplementedError("the HIP pipeline keeps FP16 buffers in float16 only")
        self.config = config
        self.layout = layout
        dev = layout.key_baseline.device
        self.device = dev
        self.boost_idx_uint8 = boost_idx_uint8.to(dev, torch.uint8).contiguous()  # (L, H, D)
        L, H, D = config.num_layers, config.num_kv_heads, config.head_dim
        S, G = config.sink_size, config.q_buffer_size
        self.num_slots = max(1, int(num_slots or config.max_batch_size))
        n = self.num_slots
        f16 = torch.float16
        self._sink_k = torch.zeros(n, L, H, S, D, dtype=f16, device=dev)
        self._sink_v = torch.zeros(n, L, H, S, D, dtype=f16, device=dev)
        self._qbuf_k = torch.zeros(n, L, H, G, D, dtype=f16, device=dev)
        self._qbuf_v = torch.zeros(n, L, H, G, D, dtype=f16, device=dev)
        self._fill = np.zeros((n, L), np.int64)     # sink tokens written
        self._qlen = np.zeros((n, L), np.int64)     # tokens in the key/value buffers
        self._npages = np.zeros((n, L), np.int64)   # pages of (slot, layer)
        self.max_pages_per_seq = (config.max_seq_len - S) // G + 2
        self._block_table = torch.zeros(L, n, self.max_pages_per_seq, dtype=torch.int32, device=dev)
        self._slot_of: Dict[int, int] = {}
        self._seq_of: Dict[int, int] = {}
        self._store = None
        if dev.type == "cuda":
            self._store = pool_store(layout.key_baseline, layout.key_boost, layout.key_metadata,
                                     layout.value_pool, layout.value_metadata)

    # ------------------------------------------------------------- slots
    def slot(self, seq_id: int) -> int:
        """Slot of a sequence, assigned (lowest free) on first use."""
        s = self._slot_of.get(seq_id)
        if s is None:
            free = [i for i in range(self.num_slots) if i not in self._seq_of]
            if not free:
                raise RuntimeError(f"all {self.num_slots} sequence slots are in use; "
                                   "raise KittyConfig.max_batch_size or reset finished sequences")
            s = free[0]
            self._slot_of[seq_id] = s
            self._seq_of[s] = seq_id
        return s

    def _slot0(self) -> int:
        return self._slot_of.get(0, 0)

    # Counters of sequence 0, layer 0: the reference's shared counters.
    @property
    def sink_fill(self) -> int:
        return int(self._fill[self._slot0(), 0])

    @property
    def key_qbuf_len(self) -> int:
        return int(self._qlen[self._slot0(), 0])

    @property
    def val_local_len(self) -> int:
        return int(self._qlen[self._slot0(), 0])

    @property
    def val_qbuf_len(self) -> int:
        return 0

    @property
    def sink_k(self) -> torch.Tensor:
        return self._sink_k[self._slot0()]

    @property
    def sink_v(self) -> torch.Tensor:
        return self._sink_v[self._slot0()]

    @property
    def key_qbuf(self) -> torch.Tensor:
        return self._qbuf_k[self._slot0()]

    @property
    def val_local(self) -> torch.Tensor:
        return self._qbuf_v[self._slot0()]

    # -------------------------------------------------------------- push
    def push_token(self, layer_id: int, key: torch.Tensor, value: torch.Tensor, seq_id: int = 0) -> None:
        """One (num_kv_heads, head_dim) token for one sequence (pipeline.py:115-181)."""
        self.push_tokens(layer_id, key.unsqueeze(0), value.unsqueeze(0), [seq_id])

    def push_tokens(self, layer_id: int, keys: torch.Tensor, values: torch.Tensor, seq_ids: Sequence[int]) -> None:
        """One token for each of B sequences: keys / values (B, num_kv_heads, head_dim)."""
        cfg = self.config
        S, G = cfg.sink_size, cfg.q_buffer_size
        slots = np.array([self.slot(s) for s in seq_ids], np.int64)
        if len(set(slots.tolist())) != len(slots):
            raise ValueError("a sequence appears twice in one push")
        keys = keys.to(self.device, torch.float16)
        values = values.to(self.device, torch.float16)
        l = layer_id
        fill = self._fill[slots, l]
        in_sink = fill < S
        if in_sink.any():
            rows = np.nonzero(in_sink)[0]
            sl = torch.as_tensor(slots[rows], device=self.device)
            pos = torch.as_tensor(fill[rows], device=self.device)
            r = torch.as_tensor(rows, device=self.device)
            self._sink_k[sl, l, :, pos] = keys[r]
            self._sink_v[sl, l, :, pos] = values[r]
            self._fill[slots[rows], l] += 1
        if (~in_sink).any():
            rows = np.nonzero(~in_sink)[0]
            qpos = self._qlen[slots[rows], l]
            sl = torch.as_tensor(slots[rows], device=self.device)
            pos = torch.as_tensor(qpos, device=self.device)
            r = torch.as_tensor(rows, device=self.device)
            self._qbuf_k[sl, l, :, pos] = keys[r]
            self._qbuf_v[sl, l, :, pos] = values[r]
            self._qlen[slots[rows], l] += 1
            full = rows[self._qlen[slots[rows], l] == G]
            if len(full):
                self._spill(l, slots[full], [seq_ids[i] for i in full])

    def _spill(self, layer: int, slots: np.ndarray, seq_ids: List[int]) -> None:
        """Quantise the full key/value buffers of these slots into one new page
        each (pipeline.py:183-256, one launch)."""
        phys = []
        for s, seq in zip(slots.tolist(), seq_ids):
            page_no = int(self._npages[s, layer])
            if page_no >= self.max_pages_per_seq:
                raise RuntimeError(f"sequence {seq} exceeds max_seq_len={self.config.max_seq_len}")
            phys.append(self.layout.allocate_page(seq, layer, page_no).physical_idx)
        if self._store is None:
            raise RuntimeError("kitty (MI355X build) quantises only on ROCm devices")
        sl = torch.as_tensor(slots, device=self.device)
        pages = torch.tensor(phys, dtype=torch.int32).to(self.device)
        kblk = self._qbuf_k[:, layer].index_select(0, sl)   # (n, H, G, D)
        vblk = self._qbuf_v[:, layer].index_select(0, sl)
        quantize_into_pools(self._store, kblk, vblk, self.boost_idx_uint8[layer], pages, self.config.sentinel)
        self._block_table[layer, sl, torch.as_tensor(self._npages[slots, layer], device=self.device)] = pages
        self._npages[slots, layer] += 1
        self._qlen[slots, layer] = 0

    # ------------------------------------------------------------- query
    def get_attention_context(self, layer_id: int, seq_id: int = 0) -> dict:
        """FP16 segments and ordered page list of one sequence (pipeline.py:260-282)."""
        s = self.slot(seq_id)
        f, q = int(self._fill[s, layer_id]), int(self._qlen[s, layer_id])
        return {
            "sink_k": self._sink_k[s, layer_id, :, :f],
            "sink_v": self._sink_v[s, layer_id, :, :f],
            "key_qbuf": self._qbuf_k[s, layer_id, :, :q],
            "val_local": self._qbuf_v[s, layer_id, :, :q],
            "page_list": self.layout.get_page_list(seq_id=seq_id, layer_id=layer_id),
        }

    def decode_inputs(self, layer_id: int, seq_ids: Sequence[int]) -> dict:
        """Batched decode operands for the sequences' slots: block table rows,
        page counts and FP16 sink / tail views with their lengths."""
        slots = np.array([self.slot(s) for s in seq_ids], np.int64)
        contiguous = bool(len(slots) and (np.diff(slots) == 1).all())
        if contiguous:
            a, b = int(slots[0]), int(slots[-1]) + 1
            pick = lambda t: t[a:b, layer_id]
        else:
            idx = torch.as_tensor(slots, device=self.device)
            pick = lambda t: t[:, layer_id].index_select(0, idx)
        lens = torch.tensor(np.stack([self._npages[slots, layer_id], self._fill[slots, layer_id],
                                      self._qlen[slots, layer_id]]), dtype=torch.int32).to(self.device)
        return dict(block_table=pick(self._block_table.transpose(0, 1)), num_pages=lens[0],
                    sink_k=pick(self._sink_k), sink_v=pick(self._sink_v), sink_len=lens[1],
                    tail_k=pick(self._qbuf_k), tail_v=pick(self._qbuf_v), tail_len=lens[2],
                    max_pages=int(self._npages[slots, layer_id].max()) if len(slots) else 0)

    # ------------------------------------------------------------- reset
    def reset_sequence(self, seq_id: int = 0) -> None:
        """Free the sequence's pages and slot (pipeline.py:286-313)."""
        self.layout.free_sequence(seq_id)
        s = self._slot_of.pop(seq_id, None)
        if s is None:
            return
        self._seq_of.pop(s, None)
        self._fill[s] = 0
        self._qlen[s] = 0
        self._npages[s] = 0
        for t in (self._sink_k, self._sink_v, self._qbuf_k, self._qbuf_v, self._block_table.transpose(0, 1)):
            t[s].zero_()

    def stats(self) -> dict:
        return {
            "sink_fill": self.sink_fill,
            "sink_capacity": self.config.sink_size,
            "key_qbuf_len": self.key_qbuf_len,
            "key_qbuf_capacity": self.config.q_buffer_size,
            "val_local_len": self.val_local_len,
            "val_local_capacity": self.config.local_value_window,
            "val_qbuf_len": self.val_qbuf_len,
            "active_sequences": len(self._slot_of),
            **self.layout.memory_stats(),
        }
