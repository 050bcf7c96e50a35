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

On a ROCm device the hot path of a decode step is:

* one ``kitty_append_tokens`` launch that writes the new token of every
  sequence of the batch into its sink or key / value buffer and advances the
  device-side counters (``lens``: sink fill, buffer length, page count per
  (layer, slot));
* for the sequences whose buffer became full, one ``kitty_quantize_kv_blocks``
  launch that packs all of them into freshly allocated pages, plus the block
  table and counter updates;
* the decode reads lengths, block table rows and FP16 segments straight from
  these device tensors.

Host state mirrors the counters (every push adds exactly one token per
sequence, so the host knows when a buffer fills without reading the device);
nothing here waits for the GPU.  A prompt (T > 1 tokens) goes through
``push_chunk``: sinks and buffer rows are copied in bulk and every complete
G-token page of the chunk is quantised straight from the chunk in one launch.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _hip
from .config import KittyConfig
from .layout import PageCentricKVLayoutManager
from .kernels.ops import pool_store, quantize_into_pools

_FILL, _QLEN, _NPAGES = 0, 1, 2


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
        # host mirrors of the counters, (slot, layer)
        self._fill = np.zeros((n, L), np.int64)     # sink tokens written
        self._qlen = np.zeros((n, L), np.int64)     # tokens in the key/value buffers
        self._npages = np.zeros((n, L), np.int64)   # pages of (slot, layer)
        # device counters (kind, layer, slot): a (layer, slot range) is a contiguous (B,) int32 view
        self.lens = torch.zeros(3, L, n, dtype=torch.int32, device=dev)
        self._overflow = torch.zeros(n, dtype=torch.int32, device=dev)
        self.max_pages_per_seq = (config.max_seq_len - S) // G + 2
        self._block_table = torch.zeros(L, n, self.max_pages_per_seq, dtype=torch.int32, device=dev)
        self._slot_of: Dict[int, int] = {}
        self._seq_of: Dict[int, int] = {}
        self._slots_dev: Dict[Tuple[int, ...], torch.Tensor] = {}
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

    def _slots_tensor(self, slots: np.ndarray) -> torch.Tensor:
        key = tuple(int(s) for s in slots)
        t = self._slots_dev.get(key)
        if t is None:
            t = torch.tensor(list(key), dtype=torch.int32).to(self.device)
            if len(self._slots_dev) > 64:
                self._slots_dev.clear()
            self._slots_dev[key] = t
        return t

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
        if self._store is not None:
            self._append_device(l, keys, values, slots)
        else:
            self._append_host(l, keys, values, slots)
        fill = self._fill[slots, l]
        in_sink = fill < S
        self._fill[slots[in_sink], l] += 1
        rows = np.nonzero(~in_sink)[0]
        self._qlen[slots[rows], l] += 1
        full = rows[self._qlen[slots[rows], l] == G]
        if len(full):
            self._spill(l, slots[full], [seq_ids[i] for i in full])

    def _append_device(self, l: int, keys: torch.Tensor, values: torch.Tensor, slots: np.ndarray) -> None:
        """kitty_append_tokens: every sequence's token into its buffers, one launch."""
        keys = keys if keys.stride(-1) == 1 else keys.contiguous()
        values = values if values.stride(-1) == 1 else values.contiguous()
        sk, sv, qk, qv = (t[:, l] for t in (self._sink_k, self._sink_v, self._qbuf_k, self._qbuf_v))
        a = _hip.AppendArgs()
        a.key, a.value = keys.data_ptr(), values.data_ptr()
        a.key_s_seq, a.key_s_head = keys.stride(0), keys.stride(1)
        a.value_s_seq, a.value_s_head = values.stride(0), values.stride(1)
        slots_dev = self._slots_tensor(slots)
        a.slots = slots_dev.data_ptr()
        a.sink_k, a.sink_v = sk.data_ptr(), sv.data_ptr()
        a.sink_layout = _hip.SlotLayout(sk.stride(0), sk.stride(1), sk.stride(2))
        a.buf_k, a.buf_v = qk.data_ptr(), qv.data_ptr()
        a.buf_layout = _hip.SlotLayout(qk.stride(0), qk.stride(1), qk.stride(2))
        a.sink_fill = self.lens[_FILL, l].data_ptr()
        a.buf_len = self.lens[_QLEN, l].data_ptr()
        a.overflow = self._overflow.data_ptr()
        a.batch, a.num_kv_heads, a.head_dim = len(slots), keys.shape[1], keys.shape[2]
        a.sink_size, a.buf_tokens, a.num_slots = self.config.sink_size, self.config.q_buffer_size, self.num_slots
        _hip.check(_hip.load().kitty_append_tokens(ctypes.byref(a), _hip.stream_ptr(self.device)))

    def _append_host(self, l: int, keys: torch.Tensor, values: torch.Tensor, slots: np.ndarray) -> None:
        """Buffer bookkeeping without a ROCm device (the FP16 buffers only;
        spilling needs the HIP kernels)."""
        S = self.config.sink_size
        fill = self._fill[slots, l]
        for i, s in enumerate(slots.tolist()):
            if fill[i] < S:
                self._sink_k[s, l, :, fill[i]] = keys[i]
                self._sink_v[s, l, :, fill[i]] = values[i]
                self.lens[_FILL, l, s] += 1
            else:
                q = int(self._qlen[s, l])
                self._qbuf_k[s, l, :, q] = keys[i]
                self._qbuf_v[s, l, :, q] = values[i]
                self.lens[_QLEN, l, s] += 1

    def overflowed(self) -> bool:
        """True if an append ever found a full, unspilled buffer (reads the device)."""
        return bool(self._overflow.any().item())

    def _alloc(self, layer: int, slot: int, seq_id: int, count: int) -> List[int]:
        first = int(self._npages[slot, layer])
        if first + count > self.max_pages_per_seq:
            raise RuntimeError(f"sequence {seq_id} exceeds max_seq_len={self.config.max_seq_len}")
        return [self.layout.allocate_page(seq_id, layer, first + i).physical_idx for i in range(count)]

    def _spill(self, layer: int, slots: np.ndarray, seq_ids: List[int]) -> None:
        """Quantise the full key/value buffers of these slots into one new page
        each (pipeline.py:183-256, one launch)."""
        phys = [self._alloc(layer, s, seq, 1)[0] for s, seq in zip(slots.tolist(), seq_ids)]
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
        self.lens[_QLEN, layer, sl] = 0
        self.lens[_NPAGES, layer, sl] += 1

    # ------------------------------------------------------------ prefill
    def push_chunk(self, layer_id: int, keys: torch.Tensor, values: torch.Tensor, seq_ids: Sequence[int]) -> None:
        """T tokens for each of B sequences at once: keys / values
        (B, num_kv_heads, T, head_dim).  The resulting state is the one T
        push_tokens calls would leave (same sinks, buffers and page contents),
        with every complete page of the chunk quantised straight from it."""
        cfg = self.config
        S, G = cfg.sink_size, cfg.q_buffer_size
        keys = keys.to(self.device, torch.float16)
        values = values.to(self.device, torch.float16)
        T = keys.shape[2]
        l = layer_id
        for i, seq in enumerate(seq_ids):
            s = self.slot(seq)
            t = 0
            f = int(self._fill[s, l])
            n_s = min(T, S - f) if f < S else 0
            if n_s:
                self._sink_k[s, l, :, f:f + n_s] = keys[i, :, :n_s]
                self._sink_v[s, l, :, f:f + n_s] = values[i, :, :n_s]
                self._fill[s, l] += n_s
                t = n_s
            q = int(self._qlen[s, l])
            if t < T and q > 0:   # top up a partly filled buffer
                n_q = min(T - t, G - q)
                self._qbuf_k[s, l, :, q:q + n_q] = keys[i, :, t:t + n_q]
                self._qbuf_v[s, l, :, q:q + n_q] = values[i, :, t:t + n_q]
                t += n_q
                self._qlen[s, l] += n_q
                self.lens[_QLEN, l, s] = int(self._qlen[s, l])
                if self._qlen[s, l] == G:
                    self._spill(l, np.array([s]), [seq])
            n_full = (T - t) // G
            if n_full:
                phys = self._alloc(l, s, seq, n_full)
                if self._store is None:
                    raise RuntimeError("kitty (MI355X build) quantises only on ROCm devices")
                blk_k = keys[i, :, t:t + n_full * G].unflatten(1, (n_full, G)).transpose(0, 1)  # (n, H, G, D)
                blk_v = values[i, :, t:t + n_full * G].unflatten(1, (n_full, G)).transpose(0, 1)
                pages = torch.tensor(phys, dtype=torch.int32).to(self.device)
                quantize_into_pools(self._store, blk_k, blk_v, self.boost_idx_uint8[l], pages, cfg.sentinel)
                p0 = int(self._npages[s, l])
                self._block_table[l, s, p0:p0 + n_full] = pages
                self._npages[s, l] += n_full
                t += n_full * G
            rem = T - t
            if rem:
                self._qbuf_k[s, l, :, :rem] = keys[i, :, t:]
                self._qbuf_v[s, l, :, :rem] = values[i, :, t:]
                self._qlen[s, l] = rem
            self.lens[:, l, s] = torch.tensor([int(self._fill[s, l]), int(self._qlen[s, l]),
                                               int(self._npages[s, l])], dtype=torch.int32).to(self.device)

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
        page counts and FP16 sink / tail views with their lengths, read from
        the device-side state (views, no copies, for a contiguous slot range)."""
        slots = np.array([self.slot(s) for s in seq_ids], np.int64)
        contiguous = bool(len(slots) and (np.diff(slots) == 1).all())
        lens = self.lens[:, layer_id]
        if contiguous:
            a, b = int(slots[0]), int(slots[-1]) + 1
            pick = lambda t: t[a:b, layer_id]
            lens = lens[:, a:b]
        else:
            idx = self._slots_tensor(slots).long()
            pick = lambda t: t[:, layer_id].index_select(0, idx)
            lens = lens.index_select(1, idx)
        return dict(block_table=pick(self._block_table.transpose(0, 1)), num_pages=lens[_NPAGES],
                    sink_k=pick(self._sink_k), sink_v=pick(self._sink_v), sink_len=lens[_FILL],
                    tail_k=pick(self._qbuf_k), tail_v=pick(self._qbuf_v), tail_len=lens[_QLEN],
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
        self.lens[:, :, s] = 0
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
