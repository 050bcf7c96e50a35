"""Token state machine of the Kitty KV cache, device-resident and batched.

Drop-in for ``KittyInferencePipeline`` (reference ``kitty/pipeline.py:49-326``):
same constructor, ``push_token``, ``get_attention_context``,
``reset_sequence``, ``stats`` and counter attributes.  Differences, all
deliberate:

* Every sequence gets its own slot of FP16 buffers and every (slot, layer) its
  own counters.  The reference keeps one shared set and advances counters only
  on layer 0 (``pipeline.py:90-111, 146-177``), so layers >= 1 and a second
  sequence overwrite each other.
* Keys and values leave FP16 on their own schedules (the KIVI split the
  reference's local value window aims at, ``pipeline.py:100-108, 155-168``):
  the keys of G buffered tokens are quantised into a new page as soon as the
  key buffer is full, the values of those same G tokens once they are older
  than the R most recent tokens.  After n tokens past the sinks a sequence
  holds P_k = n // G key pages, P_v = max(0, n - R) // G value pages (the
  value half of the same physical pages) and n - P_v G FP16 values (R to
  R + G - 1 of them once n >= R + G), so the R most recent values are always
  FP16.  Page p holds K and V of the same tokens.  The reference instead
  quantises, at each key spill, the values its window has evicted so far,
  which pairs the keys of page p with values of earlier tokens and zeros in
  page 0.  ``val_local_len`` reports the values in the R-window and
  ``val_qbuf_len`` the older FP16 values not yet quantised.  R = 0 gives the
  single-stream layout of ``paged_attention_reference`` (equal key and value
  tails, ``kernels/attention.py:163-165``).

On a ROCm device the hot path of a decode step is:

* one ``kitty_append_tokens`` launch that writes the new token of every
  sequence of the batch into its sink, key and value buffers and advances the
  device-side counters (``lens``: sink fill, key buffer length, key pages,
  value pages, value buffer length per (layer, slot));
* for the sequences whose key buffer became full, a ``kitty_quantize_kv_blocks``
  launch of their keys into freshly allocated pages; for those whose value
  buffer reached R + G rows, of their oldest G values into the value half of
  their oldest value-less page, the same launch's value blocks then moving
  the R newest values to the front of the buffer (one launch when the two
  sets are the same run of slots, as with R = G or R = 0);
* the decode reads lengths, block table rows and FP16 segments straight from
  these device tensors.

Host state mirrors the counters (every push adds exactly one token per
sequence, so the host knows when a buffer fills without reading the device);
nothing here waits for the GPU.  The few integers a spill changes on the
device (the new pages' ids, block-table entries, counters) travel in the
kernel arguments of one ``kitty_store_i32`` launch when the spilled slots are
ascending runs (every single sequence, and sequences in lockstep); other slot
sets stage their metadata through pinned memory with a non-blocking copy on
the current stream.  A prompt (T > 1 tokens) goes
through ``push_chunk``: sinks and buffer rows are copied in bulk and every
complete G-token page of the chunk is quantised straight from it.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _hip
from .config import KittyConfig
from .layout import PageCentricKVLayoutManager
from .kernels import cpu
from .kernels.ops import HostStager, QuantizePlan, pool_store, quantize_into_pools

_FILL, _QLEN, _NPAGES, _NPAGES_V, _VLEN = 0, 1, 2, 3, 4


def _is_run(slots: np.ndarray) -> bool:
    """True for a non-empty ascending run of consecutive slots."""
    return len(slots) > 0 and bool((np.diff(slots) == 1).all())


class KittyInferencePipeline:
    def __init__(self, config: KittyConfig, layout: PageCentricKVLayoutManager, boost_idx_uint8: torch.Tensor,
                 num_slots: Optional[int] = None) -> None:
        self.config = config
        self.layout = layout
        dev = layout.key_baseline.device
        self.device = dev
        self.boost_idx_uint8 = boost_idx_uint8.to(dev, torch.uint8).contiguous()  # (L, H, D)
        L, H, D = config.num_layers, config.num_kv_heads, config.head_dim
        S, G, R = config.sink_size, config.q_buffer_size, config.local_value_window
        self.num_slots = max(1, int(num_slots or config.max_batch_size))
        self.value_capacity = R + G     # FP16 values a sequence can hold before its value spill
        n = self.num_slots
        # the "FP16" buffers hold the config's dtype (pipeline.py:83-106)
        self._dtype = dt = torch.float16 if config.dtype == "float16" else torch.bfloat16
        self._sink_k = torch.zeros(n, L, H, S, D, dtype=dt, device=dev)
        self._sink_v = torch.zeros(n, L, H, S, D, dtype=dt, device=dev)
        self._qbuf_k = torch.zeros(n, L, H, G, D, dtype=dt, device=dev)
        self._vbuf = torch.zeros(n, L, H, self.value_capacity, D, dtype=dt, device=dev)
        # host mirrors of the counters, (slot, layer)
        # host copies of the five counters, one array (rows in the order of
        # self.lens) so that a batch's counters are read in one indexing
        self._counts = np.zeros((5, n, L), np.int64)
        self._fill = self._counts[_FILL]        # sink tokens written
        self._qlen = self._counts[_QLEN]        # keys in the key buffer
        self._npages = self._counts[_NPAGES]    # key pages of (slot, layer)
        self._npv = self._counts[_NPAGES_V]     # pages whose value half is written
        self._vlen = self._counts[_VLEN]        # values in the value buffer
        # device counters (kind, layer, slot): a (layer, slot range) is a contiguous (B,) int32 view
        self.lens = torch.zeros(5, L, n, dtype=torch.int32, device=dev)
        self._overflow = torch.zeros(n, dtype=torch.int32, device=dev)
        self.max_pages_per_seq = (config.max_seq_len - S) // G + 2
        self._block_table = torch.zeros(L, n, self.max_pages_per_seq, dtype=torch.int32, device=dev)
        self._pages = np.zeros((n, L, self.max_pages_per_seq), np.int64)   # host mirror of the block table
        self._slot_of: Dict[int, int] = {}
        self._seq_of: Dict[int, int] = {}
        self._slots_dev: Dict[Tuple[int, ...], torch.Tensor] = {}
        # slot arrays of batches of sequence ids seen before (cleared when a slot is freed)
        self._slots_of_ids: Dict[Tuple[int, ...], np.ndarray] = {}
        # append arguments per (layer, slots): everything but the token pointers
        self._append_args: Dict[Tuple[int, Tuple[int, ...]], Tuple[_hip.AppendArgs, torch.Tensor]] = {}
        self._lib = None
        self._stager = None         # pinned staging rows of _h2d, allocated on first use
        self._meta_dev = None       # a spill's staged metadata (fixed address, see _stage_meta)
        # per (layer, first slot, count, kind): the quantise launch of a spill
        # of that run of slots, validated once (page ids read from _meta_dev)
        self._spill_plans: Dict[Tuple[int, int, int, str], object] = {}
        # _spill_one's store list (reused)
        self._one_addrs = (ctypes.c_int64 * 8)()
        self._one_vals = (ctypes.c_int32 * 8)()
        self._on_device = dev.type == "cuda"
        if self._on_device:
            self._lib = _hip.load()
            self._store = pool_store(layout.key_baseline, layout.key_boost, layout.key_metadata,
                                     layout.value_pool, layout.value_metadata)
        else:   # pools on the CPU: spills run the torch code of kernels.cpu
            self._store = cpu.PoolSet(layout.key_baseline, layout.key_boost, layout.key_metadata,
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

    @property
    def buffer_dtype(self) -> torch.dtype:
        """torch dtype of the sink, key and value buffers (KittyConfig.dtype)."""
        return self._dtype

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
        """Values in the R-token window (pipeline.py:103)."""
        return int(min(self._vlen[self._slot0(), 0], self.config.local_value_window))

    @property
    def val_qbuf_len(self) -> int:
        """FP16 values older than the window, waiting to be quantised (pipeline.py:108)."""
        v = int(self._vlen[self._slot0(), 0])
        return v - min(v, self.config.local_value_window)

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
        """Sequence 0's FP16 value buffer, (L, H, R + G, D): the window and the
        values waiting to be quantised, oldest first."""
        return self._vbuf[self._slot0()]

    # ---------------------------------------------------- host -> device
    def _h2d(self, a, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Small int32 host data on the device without a blocking copy: a
        ring of pinned staging rows allocated once (pinning a fresh tensor
        per call cost ~75 µs of host time) and a non-blocking copy on the
        current stream into a new device tensor, or into the front of `out`
        (kernels.ops.HostStager).  A new tensor keeps the shape of `a`."""
        a = np.ascontiguousarray(a, dtype=np.int32)
        if not self._on_device:
            return torch.from_numpy(a)
        if self._stager is None:
            self._stager = HostStager(self.device, 16 + 12 * self.num_slots)
        return self._stager(a, out) if out is not None else self._stager(a).view(a.shape)

    def _slots_tensor(self, slots: np.ndarray) -> torch.Tensor:
        key = tuple(int(s) for s in slots)
        t = self._slots_dev.get(key)
        if t is None:
            t = self._h2d(np.array(key, np.int32))
            if len(self._slots_dev) > 64:
                self._slots_dev.clear()
            self._slots_dev[key] = t
        return t

    # -------------------------------------------------------------- push
    def push_token(self, layer_id: int, key: torch.Tensor, value: torch.Tensor, seq_id: int = 0) -> None:
        """One (num_kv_heads, head_dim) token for one sequence (pipeline.py:115-181)."""
        self.push_tokens(layer_id, key.unsqueeze(0), value.unsqueeze(0), [seq_id])

    def push_tokens(self, layer_id: int, keys: torch.Tensor, values: torch.Tensor, seq_ids: Sequence[int]) -> None:
        """One token for each of B sequences: keys / values (B, num_kv_heads, head_dim)."""
        cfg = self.config
        S, G = cfg.sink_size, cfg.q_buffer_size
        ids = tuple(seq_ids)
        slots = self._slots_of_ids.get(ids)
        if slots is None:
            slots = np.array([self.slot(s) for s in ids], np.int64)
            if len(set(slots.tolist())) != len(slots):
                raise ValueError("a sequence appears twice in one push")
            if len(self._slots_of_ids) >= 256:
                self._slots_of_ids.clear()
            self._slots_of_ids[ids] = slots
        keys = keys.to(self.device, self._dtype)
        values = values.to(self.device, self._dtype)
        l = layer_id
        append = self._append_device if self._on_device else self._append_host
        if len(slots) == 1:
            # one sequence (push_token): the same steps on scalar counters
            s = int(slots[0])
            in_sink = self._fill[s, l] < S
            kf = not in_sink and self._qlen[s, l] + 1 == G
            vf = not in_sink and self._vlen[s, l] + 1 == self.value_capacity
            phys = []
            if kf:      # _alloc_spill for one page of one sequence
                pno = int(self._npages[s, l])
                if pno + 1 > self.max_pages_per_seq:
                    raise RuntimeError(f"sequence {ids[0]} exceeds max_seq_len={cfg.max_seq_len}")
                phys = self.layout.allocate_run(ids[0], l, pno, 1)
            append(l, keys, values, slots)
            if in_sink:
                self._fill[s, l] += 1
            else:
                self._qlen[s, l] += 1
                self._vlen[s, l] += 1
            if kf or vf:
                if self._on_device and cfg.local_value_window <= G:
                    self._spill_one(l, s, kf, vf, phys)
                else:
                    self._spill(l, slots if kf else slots[:0], phys, slots if vf else slots[:0])
            return
        fill = self._fill[slots, l]
        in_sink = fill < S
        rows = np.nonzero(~in_sink)[0]
        # sequences whose buffers this token fills: their new pages are taken
        # first, all or nothing, so a full pool raises before any state changes
        kfull = rows[self._qlen[slots[rows], l] + 1 == G]
        vfull = rows[self._vlen[slots[rows], l] + 1 == self.value_capacity]
        phys = self._alloc_spill(l, slots[kfull], [seq_ids[i] for i in kfull]) if len(kfull) else []
        append(l, keys, values, slots)
        self._fill[slots[in_sink], l] += 1
        self._qlen[slots[rows], l] += 1
        self._vlen[slots[rows], l] += 1
        if len(kfull) or len(vfull):
            self._spill(l, slots[kfull], phys, slots[vfull])

    def _append_device(self, l: int, keys: torch.Tensor, values: torch.Tensor, slots: np.ndarray) -> None:
        """kitty_append_tokens: every sequence's token into its buffers, one launch."""
        keys = keys if keys.stride(-1) == 1 else keys.contiguous()
        values = values if values.stride(-1) == 1 else values.contiguous()
        ck = (l, tuple(slots.tolist()))
        hit = self._append_args.get(ck)
        if hit is None:
            hit = self._append_args[ck] = self._append_setup(l, slots, keys.shape[1], keys.shape[2])
            if len(self._append_args) > 256:
                self._append_args.clear()
                self._append_args[ck] = hit
        a = hit[0]
        a.key, a.value = keys.data_ptr(), values.data_ptr()
        a.key_s_seq, a.key_s_head = keys.stride(0), keys.stride(1)
        a.value_s_seq, a.value_s_head = values.stride(0), values.stride(1)
        _hip.check(self._lib.kitty_append_tokens(ctypes.byref(a), _hip.stream_ptr(self.device)))

    def _append_setup(self, l: int, slots: np.ndarray, H: int, D: int) -> Tuple[_hip.AppendArgs, torch.Tensor]:
        """kitty_append_tokens arguments of layer l for these slots, bar the
        token pointers and strides (the buffers and counters never move), with
        the slot-id tensor they point at."""
        sk, sv, qk, vb = (t[:, l] for t in (self._sink_k, self._sink_v, self._qbuf_k, self._vbuf))
        a = _hip.AppendArgs()
        slots_dev = self._slots_tensor(slots)
        a.slots = slots_dev.data_ptr()
        a.sink_k, a.sink_v = sk.data_ptr(), sv.data_ptr()
        a.sink_layout = _hip.SlotLayout(sk.stride(0), sk.stride(1), sk.stride(2))
        a.buf_k = qk.data_ptr()
        a.buf_layout = _hip.SlotLayout(qk.stride(0), qk.stride(1), qk.stride(2))
        a.sink_fill = self.lens[_FILL, l].data_ptr()
        a.buf_len = self.lens[_QLEN, l].data_ptr()
        a.val_len = self.lens[_VLEN, l].data_ptr()
        a.val_buf = vb.data_ptr()
        a.val_layout = _hip.SlotLayout(vb.stride(0), vb.stride(1), vb.stride(2))
        a.val_tokens = self.value_capacity
        a.overflow = self._overflow.data_ptr()
        a.batch, a.num_kv_heads, a.head_dim = len(slots), H, D
        a.sink_size, a.buf_tokens, a.num_slots = self.config.sink_size, self.config.q_buffer_size, self.num_slots
        return a, slots_dev

    def _append_host(self, l: int, keys: torch.Tensor, values: torch.Tensor, slots: np.ndarray) -> None:
        """The token append for buffers on the CPU: the same routing as
        kitty_append_tokens (sink while it has room, else key and value
        buffers), one sequence at a time."""
        S = self.config.sink_size
        fill = self._fill[slots, l]
        for i, s in enumerate(slots.tolist()):
            if fill[i] < S:
                self._sink_k[s, l, :, fill[i]] = keys[i]
                self._sink_v[s, l, :, fill[i]] = values[i]
                self.lens[_FILL, l, s] += 1
            else:
                self._qbuf_k[s, l, :, int(self._qlen[s, l])] = keys[i]
                self._vbuf[s, l, :, int(self._vlen[s, l])] = values[i]
                self.lens[_QLEN, l, s] += 1
                self.lens[_VLEN, l, s] += 1

    def overflowed(self) -> bool:
        """True if an append ever found a full, unspilled buffer (reads the device)."""
        return bool(self._overflow.any().item())

    def _alloc_spill(self, layer: int, slots: np.ndarray, seq_ids: Sequence[int],
                     counts: Optional[Sequence[int]] = None) -> List[int]:
        """Physical pages for the next key pages of these sequences (counts[i]
        of them, default one each), all or nothing: on a full pool or a
        sequence past max_seq_len the pages already taken are returned and
        RuntimeError is raised."""
        taken: List[Tuple[int, int, List[int]]] = []   # (seq, first page number, its run)
        try:
            for i, (s, seq) in enumerate(zip(np.asarray(slots).tolist(), seq_ids)):
                first = int(self._npages[s, layer])
                count = 1 if counts is None else int(counts[i])
                if first + count > self.max_pages_per_seq:
                    raise RuntimeError(f"sequence {seq} exceeds max_seq_len={self.config.max_seq_len}")
                taken.append((seq, first, self.layout.allocate_run(seq, layer, first, count)))
        except RuntimeError:
            for seq, first, run in taken:
                for j in range(len(run)):
                    self.layout.free_page(seq, layer, first + j)
            raise
        return [ph for _, _, run in taken for ph in run]

    def _spill(self, layer: int, kslots: np.ndarray, phys: List[int], vslots: np.ndarray) -> None:
        """Key spill of kslots (their full key buffers into the new pages
        phys, one each) and value spill of vslots (the oldest G values into
        the value half of their first value-less page, then the R newest
        values to the front of the buffer) (pipeline.py:183-256).  The host
        counters are advanced first.

        On the device, when both slot sets are ascending runs (sequences that
        advance in lockstep, and every single sequence) and R <= G, the work
        is _spill_runs: the new ids, block-table entries and counters in one
        kitty_store_i32 launch and the quantise launches cached per (layer,
        run), the value window's shift inside the value launch.  Otherwise
        (other slot sets, R > G, CPU pools) the new counters, slots and page
        ids go to the device in one pinned copy; the blocks are gathered, and
        the block table, counters and value shift are indexed torch writes."""
        G, R = self.config.q_buffer_size, self.config.local_value_window
        both = R == 0
        k, v = len(kslots), (0 if both else len(vslots))
        n = self.num_slots
        pno = self._npages[kslots, layer].copy()
        vphys = self._pages[vslots, layer, self._npv[vslots, layer]] if v else np.zeros(0, np.int64)
        if k:
            self._pages[kslots, layer, pno] = phys
            self._npages[kslots, layer] += 1
            self._qlen[kslots, layer] = 0
            if both:
                self._npv[kslots, layer] += 1
                self._vlen[kslots, layer] = 0
        if v:
            self._npv[vslots, layer] += 1
            self._vlen[vslots, layer] -= G
        if v == 0:
            touched = np.asarray(kslots, np.int64)
        elif k == 0 or (k == v and np.array_equal(kslots, vslots)):
            touched = np.asarray(vslots[:v], np.int64)
        else:
            touched = np.union1d(kslots, vslots[:v]).astype(np.int64)
        if self._on_device and R <= G and (k == 0 or _is_run(kslots)) and (v == 0 or _is_run(vslots[:v])):
            self._spill_runs(layer, kslots, np.asarray(phys, np.int64), pno, vslots[:v], vphys, touched, both)
            return
        lens_new = self._counts[:, touched, layer]
        nt = len(touched)
        # staged int32: key page ids at [0, k), value page ids at [n, n + v)
        # (fixed places the cached launches read), then slots, page numbers
        # and the touched slots' counters
        host = np.zeros(2 * n + 3 * k + v + 6 * nt, np.int64)
        host[:k] = phys
        host[n:n + v] = vphys
        o = 2 * n
        for part in (kslots, pno, vslots[:v], touched, lens_new.ravel()):
            host[o:o + len(part)] = part
            o += len(part)
        meta = self._stage_meta(host)
        kpages, vpages = meta[:k], meta[n:n + v]
        o = 2 * n
        ksl, kpn = meta[o:o + k], meta[o + k:o + 2 * k]
        vsl = meta[o + 2 * k:o + 2 * k + v]
        o += 2 * k + v
        tsl, lens_dev = meta[o:o + nt], meta[o + nt:o + 6 * nt].view(5, nt)
        sentinel = self.config.sentinel
        if k:
            if _is_run(kslots):
                a = int(kslots[0])
                if self._on_device:
                    self._run_plan(layer, a, k, "kv" if both else "k", meta).run()
                else:
                    quantize_into_pools(self._store, self._qbuf_k[a:a + k, layer],
                                        self._vbuf[a:a + k, layer, :, :G] if both else None,
                                        self.boost_idx_uint8[layer], kpages, sentinel)
                if (pno == pno[0]).all():   # sequences in lockstep: one page number
                    self._block_table[layer, a:a + k, int(pno[0])] = kpages if k > 1 else int(phys[0])
                else:
                    self._block_table[layer, ksl, kpn] = kpages
            else:
                kblk = self._qbuf_k[:, layer].index_select(0, ksl)
                vblk = self._vbuf[:, layer].index_select(0, ksl)[:, :, :G] if both else None
                quantize_into_pools(self._store, kblk, vblk, self.boost_idx_uint8[layer], kpages, sentinel)
                self._block_table[layer, ksl, kpn] = kpages
        if v:
            vb = self._vbuf[:, layer]                                     # (slots, H, R + G, D)
            if _is_run(vslots[:v]):
                a = int(vslots[0])
                vblk = vb[a:a + v]
                if self._on_device:
                    self._run_plan(layer, a, v, "v", meta).run()
                else:
                    quantize_into_pools(self._store, None, vblk[:, :, :G], None, vpages, sentinel)
                if R:   # the R newest values move to the front, after the launch above read the oldest G
                    src = vblk[:, :, G:G + R]
                    vblk[:, :, :R] = src if R <= G else src.clone()       # overlapping rows need a copy first
            else:
                vblk = vb.index_select(0, vsl)                            # a copy: the shift below reuses rows
                quantize_into_pools(self._store, None, vblk[:, :, :G], None, vpages, sentinel)
                if R:
                    vb[vsl, :, :R] = vblk[:, :, G:G + R]                  # the R newest values move to the front
        if _is_run(touched):
            self.lens[:, layer, int(touched[0]):int(touched[0]) + nt] = lens_dev
        else:
            self.lens[:, layer, tsl] = lens_dev

    def _spill_runs(self, layer: int, kslots: np.ndarray, phys: np.ndarray, pno: np.ndarray, vslots: np.ndarray,
                    vphys: np.ndarray, touched: np.ndarray, both: bool) -> None:
        """The device side of a spill whose key and value slots are ascending
        runs (every single sequence, and sequences in lockstep), with R <= G:
        one kitty_store_i32 launch writes the page ids the cached quantise
        launches read, the new block-table entries and the touched slots'
        counters, all carried in its kernel arguments (no staging copy);
        then one quantise launch for keys and values of the same run (key
        pages and value pages of their own), or one each, whose value blocks
        also move the window's R newest values to the front of the value
        buffer after reading the oldest G (kitty_quant_batch.value_shift)."""
        cfg = self.config
        G, R = cfg.q_buffer_size, cfg.local_value_window
        n, L, maxp = self.num_slots, cfg.num_layers, self.max_pages_per_seq
        k, v, nt = len(kslots), len(vslots), len(touched)
        if self._meta_dev is None:
            self._meta_dev = torch.zeros(16 + 12 * n, dtype=torch.int32, device=self.device)
        meta = self._meta_dev
        mp, bp, lp = meta.data_ptr(), self._block_table.data_ptr(), self.lens.data_ptr()
        addrs = np.empty(2 * k + v + 5 * nt, np.int64)
        vals = np.empty(len(addrs), np.int32)
        addrs[:k] = mp + 4 * np.arange(k)
        vals[:k] = phys
        addrs[k:k + v] = mp + 4 * (n + np.arange(v))
        vals[k:k + v] = vphys
        addrs[k + v:2 * k + v] = bp + 4 * ((layer * n + np.asarray(kslots, np.int64)) * maxp + pno)
        vals[k + v:2 * k + v] = phys
        addrs[2 * k + v:] = (lp + 4 * ((np.arange(5)[:, None] * L + layer) * n + touched[None, :])).ravel()
        vals[2 * k + v:] = self._counts[:, touched, layer].ravel()
        _hip.check(self._lib.kitty_store_i32(addrs.ctypes.data, vals.ctypes.data, len(addrs),
                                             _hip.stream_ptr(self.device)))
        if k and v and k == v and kslots[0] == vslots[0]:     # the same run: one launch for keys and values
            self._run_plan(layer, int(kslots[0]), k, "kvs", meta).run()
            return
        if k:
            self._run_plan(layer, int(kslots[0]), k, "kv" if both else "k", meta).run()
        if v:
            self._run_plan(layer, int(vslots[0]), v, "vs" if R else "v", meta).run()

    def _spill_one(self, layer: int, s: int, kf: bool, vf: bool, phys: List[int]) -> None:
        """_spill_runs for one sequence (slot s), on Python scalars: the
        same host counter updates and the same two launches, with the store
        list built in reused ctypes arrays."""
        cfg = self.config
        G, R = cfg.q_buffer_size, cfg.local_value_window
        both = R == 0
        n, L = self.num_slots, cfg.num_layers
        if self._meta_dev is None:
            self._meta_dev = torch.zeros(16 + 12 * n, dtype=torch.int32, device=self.device)
        meta = self._meta_dev
        addrs, vals = self._one_addrs, self._one_vals
        mp = meta.data_ptr()
        m = 0
        if kf:
            page = int(phys[0])
            pno = int(self._npages[s, layer])
            self._pages[s, layer, pno] = page
            self._npages[s, layer] = pno + 1
            self._qlen[s, layer] = 0
            addrs[0], vals[0] = mp, page
            addrs[1] = self._block_table.data_ptr() + 4 * ((layer * n + s) * self.max_pages_per_seq + pno)
            vals[1] = page
            m = 2
            if both:
                self._npv[s, layer] += 1
                self._vlen[s, layer] = 0
        vf = vf and not both
        if vf:
            npv = int(self._npv[s, layer])
            addrs[m], vals[m] = mp + 4 * n, int(self._pages[s, layer, npv])
            m += 1
            self._npv[s, layer] = npv + 1
            self._vlen[s, layer] -= G
        lp = self.lens.data_ptr() + 4 * (layer * n + s)
        for c in range(5):
            addrs[m + c] = lp + 4 * c * L * n
            vals[m + c] = int(self._counts[c, s, layer])
        _hip.check(self._lib.kitty_store_i32(addrs, vals, m + 5, _hip.stream_ptr(self.device)))
        kind = ("kvs" if vf else "k") if kf and not both else ("kv" if kf else ("vs" if R else "v"))
        self._run_plan(layer, s, 1, kind, meta).run()

    def _stage_meta(self, host: np.ndarray) -> torch.Tensor:
        """A spill's int32 metadata on the device, in a buffer of fixed
        address (the cached launches of _run_plan read their page ids from
        it), copied straight from the pinned staging ring; stream order keeps
        a spill's copy behind the previous spill's launches that read it."""
        if not self._on_device:
            return self._h2d(host)
        if self._meta_dev is None:
            self._meta_dev = torch.zeros(16 + 12 * self.num_slots, dtype=torch.int32, device=self.device)
        self._h2d(host, out=self._meta_dev)
        return self._meta_dev

    def _run_plan(self, layer: int, a: int, count: int, kind: str, meta: torch.Tensor):
        """The quantise launch of a spill of slots [a, a + count) at a layer,
        validated once and kept: "k" (keys into the pages at meta[0:count]),
        "kv" (keys and values into those pages, R = 0), "v" (values into the
        pages at meta[n:n + count]), "vs" (the same, then the R-row window
        shift of each value block) or "kvs" (keys into meta[0:count], values
        into meta[n:n + count], then the shift)."""
        key = (layer, a, count, kind)
        plan = self._spill_plans.get(key)
        if plan is None:
            G, n, R = self.config.q_buffer_size, self.num_slots, self.config.local_value_window
            kb = self._qbuf_k[a:a + count, layer] if kind in ("k", "kv", "kvs") else None
            vb = self._vbuf[a:a + count, layer, :, :G] if kind != "k" else None
            ids = meta[n:n + count] if kind in ("v", "vs") else meta[:count]
            plan = QuantizePlan(self._store, kb, vb, self.boost_idx_uint8[layer] if kb is not None else None, ids,
                                self.config.sentinel, value_page_ids=meta[n:n + count] if kind == "kvs" else None,
                                value_shift=R if kind in ("vs", "kvs") else 0)
            if len(self._spill_plans) >= 256:
                self._spill_plans.clear()
            self._spill_plans[key] = plan
        return plan

    # ------------------------------------------------------------ prefill
    def push_chunk(self, layer_id: int, keys: torch.Tensor, values: torch.Tensor, seq_ids: Sequence[int]) -> None:
        """T tokens for each of B sequences at once: keys / values
        (B, num_kv_heads, T, head_dim).  The resulting state is the one T
        push_tokens calls would leave (same sinks, buffers and page contents),
        with every complete page of the chunk quantised straight from it."""
        cfg = self.config
        S, G, R = cfg.sink_size, cfg.q_buffer_size, cfg.local_value_window
        keys = keys.to(self.device, self._dtype)
        values = values.to(self.device, self._dtype)
        T = keys.shape[2]
        l = layer_id
        slots = np.array([self.slot(seq) for seq in seq_ids], dtype=np.int64)
        if len(set(slots.tolist())) != len(slots):
            raise ValueError("a sequence appears twice in one push")
        if not self._counts[:, slots, l].any():
            self._push_chunk_fresh(l, keys, values, slots, seq_ids)
            return
        # every sequence's new key pages, all or nothing, before any state
        # changes: a full pool raises with the batch untouched
        fills = self._fill[slots, l]
        n_sink = np.where(fills < S, np.minimum(T, S - fills), 0)
        n_fulls = np.where(T > n_sink, (self._qlen[slots, l] + T - n_sink) // G, 0)
        need = np.nonzero(n_fulls)[0]
        phys_all = self._alloc_spill(l, slots[need], [seq_ids[i] for i in need], n_fulls[need]) if len(need) else []
        runs = np.split(np.asarray(phys_all, np.int64), np.cumsum(n_fulls[need])[:-1]) if len(need) else []
        phys_of = dict(zip(need.tolist(), runs))
        for i, seq in enumerate(seq_ids):
            s = int(slots[i])
            t = 0
            f = int(self._fill[s, l])
            n_s, n_full = int(n_sink[i]), int(n_fulls[i])
            phys = phys_of.get(i, [])
            if n_s:
                self._sink_k[s, l, :, f:f + n_s] = keys[i, :, :n_s]
                self._sink_v[s, l, :, f:f + n_s] = values[i, :, :n_s]
                self._fill[s, l] += n_s
                t = n_s
            m = T - t
            if m:
                # keys: buffered keys + the chunk, cut into full pages and a new buffer
                nk = int(self._qlen[s, l])
                kall = torch.cat([self._qbuf_k[s, l, :, :nk], keys[i, :, t:]], dim=1)   # (H, nk + m, D)
                if n_full:
                    p0 = int(self._npages[s, l])
                    self._pages[s, l, p0:p0 + n_full] = phys
                    pages = self._h2d(np.asarray(phys))
                    blk_k = kall[:, :n_full * G].unflatten(1, (n_full, G)).transpose(0, 1)   # (n, H, G, D)
                    vblk = None
                    if R == 0:   # values leave FP16 with their keys
                        nv = int(self._vlen[s, l])
                        vall = torch.cat([self._vbuf[s, l, :, :nv], values[i, :, t:]], dim=1)
                        vblk = vall[:, :n_full * G].unflatten(1, (n_full, G)).transpose(0, 1)
                    quantize_into_pools(self._store, blk_k, vblk, self.boost_idx_uint8[l], pages, cfg.sentinel)
                    self._block_table[l, s, p0:p0 + n_full] = pages
                    self._npages[s, l] += n_full
                    if R == 0:
                        self._npv[s, l] += n_full
                rem = nk + m - n_full * G
                self._qbuf_k[s, l, :, :rem] = kall[:, n_full * G:]
                self._qlen[s, l] = rem
                # values: buffered values + the chunk; full pages spill while
                # more than R values would stay behind
                nv = int(self._vlen[s, l])
                vall = torch.cat([self._vbuf[s, l, :, :nv], values[i, :, t:]], dim=1)        # (H, nv + m, D)
                if R == 0:
                    v_full = n_full
                else:
                    v_full = max(0, (nv + m - R) // G)
                    if v_full:
                        pv0 = int(self._npv[s, l])
                        pages_v = self._h2d(self._pages[s, l, pv0:pv0 + v_full])
                        blk_v = vall[:, :v_full * G].unflatten(1, (v_full, G)).transpose(0, 1)
                        quantize_into_pools(self._store, None, blk_v, None, pages_v, cfg.sentinel)
                        self._npv[s, l] += v_full
                vrem = nv + m - v_full * G
                self._vbuf[s, l, :, :vrem] = vall[:, v_full * G:]
                self._vlen[s, l] = vrem
            self.lens[:, l, s] = self._h2d(self._counts[:, s, l])

    def _push_chunk_fresh(self, l: int, keys: torch.Tensor, values: torch.Tensor, slots: np.ndarray,
                          seq_ids: Sequence[int]) -> None:
        """push_chunk for sequences that hold nothing yet at layer l (a new
        prompt), batched over the sequences: the same state as the
        per-sequence path, from one copy per buffer kind, one key-page and one
        value-page quantise launch for all of them (reading the pages in place
        from the prompt tensors), and one counter write."""
        cfg = self.config
        S, G, R = cfg.sink_size, cfg.q_buffer_size, cfg.local_value_window
        B, H, T, D = keys.shape
        n_s = min(T, S)
        m = T - n_s
        n_full = m // G                                     # key pages of every sequence
        v_full = n_full if R == 0 else max(0, (m - R) // G)  # of them, pages whose value half fills now
        rem, vrem = m - n_full * G, m - v_full * G
        phys = self._alloc_spill(l, slots, seq_ids, [n_full] * B) if n_full else []   # all or nothing
        # one ascending run of slots (the usual case) is written through a
        # slice: plain strided copies instead of indexed scatters
        sl = slice(int(slots[0]), int(slots[0]) + B) if _is_run(slots) else self._slots_tensor(slots).long()
        if n_s:
            self._sink_k[sl, l, :, :n_s] = keys[:, :, :n_s]
            self._sink_v[sl, l, :, :n_s] = values[:, :, :n_s]

        def blocks(x: torch.Tensor, n: int) -> torch.Tensor:       # (B, n, H, G, D) view of the prompt's pages
            return x[:, :, n_s:n_s + n * G].unflatten(2, (n, G)).transpose(1, 2)

        if n_full:
            phys = np.asarray(phys, np.int32)
            pages = self._h2d(phys)                                  # sequence-major: b * n_full + p
            quantize_into_pools(self._store, blocks(keys, n_full), blocks(values, n_full) if R == 0 else None,
                                self.boost_idx_uint8[l], pages, cfg.sentinel)
            self._block_table[l, sl, :n_full] = pages.view(B, n_full)
            self._pages[slots, l, :n_full] = phys.reshape(B, n_full)
            if R and v_full:
                pages_v = pages.view(B, n_full)[:, :v_full].reshape(-1)
                quantize_into_pools(self._store, None, blocks(values, v_full), None, pages_v, cfg.sentinel)
        if rem:
            self._qbuf_k[sl, l, :, :rem] = keys[:, :, n_s + n_full * G:]
        if vrem:
            self._vbuf[sl, l, :, :vrem] = values[:, :, n_s + v_full * G:]
        self._fill[slots, l] = n_s
        self._qlen[slots, l] = rem
        self._npages[slots, l] = n_full
        self._npv[slots, l] = v_full
        self._vlen[slots, l] = vrem
        self.lens[:, l, sl] = self._h2d(self._counts[:, slots, l])

    # ------------------------------------------------------------- query
    def get_attention_context(self, layer_id: int, seq_id: int = 0) -> dict:
        """FP16 segments and ordered page list of one sequence
        (pipeline.py:260-282): the key pages, the FP16 key buffer, and the
        FP16 values not yet in pages (val_local: the values of the last
        value_pages * G ... n tokens, oldest first) with the number of pages
        whose value half holds values (value_pages)."""
        s = self.slot(seq_id)
        f, q, v = int(self._fill[s, layer_id]), int(self._qlen[s, layer_id]), int(self._vlen[s, layer_id])
        return {
            "sink_k": self._sink_k[s, layer_id, :, :f],
            "sink_v": self._sink_v[s, layer_id, :, :f],
            "key_qbuf": self._qbuf_k[s, layer_id, :, :q],
            "val_local": self._vbuf[s, layer_id, :, :v],
            "page_list": self.layout.get_page_list(seq_id=seq_id, layer_id=layer_id),
            "value_pages": int(self._npv[s, layer_id]),
        }

    def decode_inputs(self, layer_id: int, seq_ids: Sequence[int], full_width: bool = False) -> dict:
        """Batched decode operands for the sequences' slots: block table rows,
        key / value page counts and FP16 sink / key-tail / value-tail views
        with their lengths, read from the device-side state (views, no
        copies, for a contiguous slot range: then `contiguous` is True and
        the views stay valid for later steps).  With R = 0 the value stream is
        the key stream's (num_pages_v / tail_len_v None).  max_pages is the
        batch's largest page count, or the table width with full_width."""
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
        split = self.config.local_value_window > 0
        if full_width:
            max_pages = self.max_pages_per_seq
        else:
            max_pages = int(self._npages[slots, layer_id].max()) if len(slots) else 0
        return dict(block_table=pick(self._block_table.transpose(0, 1)), num_pages=lens[_NPAGES],
                    sink_k=pick(self._sink_k), sink_v=pick(self._sink_v), sink_len=lens[_FILL],
                    tail_k=pick(self._qbuf_k), tail_v=pick(self._vbuf), tail_len=lens[_QLEN],
                    num_pages_v=lens[_NPAGES_V] if split else None, tail_len_v=lens[_VLEN] if split else None,
                    max_pages=max_pages, contiguous=contiguous)

    # ------------------------------------------------------------- reset
    def reset_sequence(self, seq_id: int = 0) -> None:
        """Free the sequence's pages and slot (pipeline.py:286-313)."""
        self.layout.free_sequence(seq_id)
        s = self._slot_of.pop(seq_id, None)
        if s is None:
            return
        self._seq_of.pop(s, None)
        self._slots_of_ids.clear()
        for c in (self._fill, self._qlen, self._npages, self._npv, self._vlen):
            c[s] = 0
        self._pages[s] = 0
        self.lens[:, :, s] = 0
        for t in (self._sink_k, self._sink_v, self._qbuf_k, self._vbuf, self._block_table.transpose(0, 1)):
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
