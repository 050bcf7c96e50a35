"""Torch-facing wrappers over the C ABI (include/kitty_hip.h).

Every function here validates shapes/dtypes/devices on the host, builds the
plain-C argument structs from tensor pointers and strides, and launches on the
caller's current HIP stream.  CPU tensors are dispatched by device to the
torch code of ``kernels.cpu`` (:func:`quantize_into_pools` with a
``cpu.PoolSet``, :func:`decode_plan`); device tensors only ever reach the
HIP library.
"""
from __future__ import annotations

import collections
import ctypes
import math
import warnings
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

from .. import _hip
from . import cpu


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dtype16(name: str, *tensors: torch.Tensor) -> int:
    """KITTY_DTYPE_* shared by tensors that must all be float16 or all
    bfloat16 (KittyConfig.dtype, config.py:76)."""
    codes = {_hip.dtype_code(t, name) for t in tensors if t is not None}
    _need(len(codes) == 1, f"{name} must all be float16 or all bfloat16")
    return codes.pop()


def _dev_i32(values: Sequence[int], device: torch.device) -> torch.Tensor:
    return torch.tensor(list(values), dtype=torch.int32).to(device, non_blocking=True)


# ------------------------------------------------------------ page stores

def pool_store(key_baseline: torch.Tensor, key_boost: torch.Tensor, key_meta: torch.Tensor,
               value_pool: torch.Tensor, value_meta: torch.Tensor) -> _hip.PageStore:
    """PageStore over the layout manager's five (P, H, ...) pools."""
    P, H, D, G4 = key_baseline.shape
    G = G4 * 4
    Dk = key_boost.shape[2]
    _need(key_baseline.dtype == torch.uint8 and key_boost.dtype == torch.uint8 and value_pool.dtype == torch.uint8,
          "packed pools must be uint8")
    meta_dtype = _dtype16("key_metadata and value_metadata", key_meta, value_meta)
    _need(tuple(key_boost.shape[:2]) == (P, H) and key_boost.shape[3] == G4, "key_boost shape")
    _need(tuple(key_meta.shape) == (P, H, 2, D), "key_metadata shape")
    _need(tuple(value_pool.shape) == (P, H, G, D // 4), "value_pool shape")
    _need(tuple(value_meta.shape) == (P, H, G, 2), "value_metadata shape")
    for t in (key_baseline, key_boost, value_pool):
        _need(t.stride(3) == 1, "packed pools need a contiguous last dimension")
    s = _hip.PageStore()
    s.key_low = key_baseline.data_ptr()
    s.key_low_s_page, s.key_low_s_head, s.key_low_s_row = key_baseline.stride()[:3]
    s.key_high = key_boost.data_ptr() if Dk > 0 else 0
    s.key_high_s_page, s.key_high_s_head, s.key_high_s_row = key_boost.stride()[:3]
    s.key_scale = key_meta.data_ptr()
    s.key_zero = key_meta.data_ptr() + key_meta.stride(2) * 2
    s.key_meta_s_page, s.key_meta_s_head = key_meta.stride(0), key_meta.stride(1)
    s.key_meta_s_chan = key_meta.stride(3)
    s.value = value_pool.data_ptr()
    s.value_s_page, s.value_s_head, s.value_s_row = value_pool.stride()[:3]
    s.value_scale = value_meta.data_ptr()
    s.value_zero = value_meta.data_ptr() + value_meta.stride(3) * 2
    s.value_meta_s_page, s.value_meta_s_head, s.value_meta_s_tok = value_meta.stride()[:3]
    s.num_pages = P
    s.num_kv_heads, s.head_dim, s.page_tokens, s.d_boost = H, D, G, Dk
    s.meta_dtype = meta_dtype
    return s


def _quant_batch(store: _hip.PageStore, key: Optional[torch.Tensor], value: Optional[torch.Tensor],
                 boost_idx: Optional[torch.Tensor], page_ids: torch.Tensor, sentinel: int,
                 value_rows: Optional[int], value_page_ids: Optional[torch.Tensor] = None,
                 value_shift: int = 0) -> Tuple[_hip.QuantBatch, torch.device]:
    ref = key if key is not None else value
    _need(ref is not None, "nothing to quantise")
    dev = _hip.require_device(key, value, boost_idx, page_ids, value_page_ids)
    _need(ref.dim() in (4, 5), "key / value blocks must be (n_outer, H, G, D) or (n_seq, pages, H, G, D)")
    per_seq = ref.shape[1] if ref.dim() == 5 else 0
    n_outer = ref.shape[0] * per_seq if per_seq else ref.shape[0]
    n_inner, G, D = ref.shape[-3:]
    _need(G == store.page_tokens and D == store.head_dim and n_inner == store.num_kv_heads,
          "block shape does not match the pools")
    _need(page_ids.dtype == torch.int32 and page_ids.numel() == n_outer, "page_ids must be int32 (n_outer,)")
    b = _hip.QuantBatch()
    b.src_dtype = _dtype16("key and value blocks", key, value)
    b.outer_per_seq = per_seq
    if key is not None:
        _need(key.shape == ref.shape, "key shape")
        b.key = key.data_ptr()
        if per_seq:
            b.key_s_seq, b.key_s_outer, b.key_s_inner, b.key_s_tok, b.key_s_chan = key.stride()
        else:
            b.key_s_outer, b.key_s_inner, b.key_s_tok, b.key_s_chan = key.stride()
    if value is not None:
        _need(value.shape == ref.shape, "value shape")
        b.value = value.data_ptr()
        if per_seq:
            b.value_s_seq, b.value_s_outer, b.value_s_inner, b.value_s_tok, b.value_s_chan = value.stride()
        else:
            b.value_s_outer, b.value_s_inner, b.value_s_tok, b.value_s_chan = value.stride()
    if key is not None:
        _need(boost_idx is not None and boost_idx.dtype == torch.uint8 and boost_idx.shape[-1] == D
              and boost_idx.stride(-1) == 1, "boost_idx must be uint8 (..., D) with contiguous rows")
        _need(tuple(boost_idx.shape[:-1]) in ((n_outer, n_inner), (n_inner,)),
              "boost_idx must be (n_outer, H, D) or (H, D)")
        b.boost_idx = boost_idx.data_ptr()
        if boost_idx.dim() == 3:
            b.boost_s_outer, b.boost_s_inner = boost_idx.stride(0), boost_idx.stride(1)
        else:
            b.boost_s_outer, b.boost_s_inner = 0, boost_idx.stride(0)
    b.page_ids = page_ids.data_ptr()
    b.n_outer, b.n_inner = n_outer, n_inner
    b.value_rows = G if value_rows is None else int(value_rows)
    b.sentinel = int(sentinel)
    if value_page_ids is not None:
        _need(value is not None and value_page_ids.dtype == torch.int32 and value_page_ids.numel() == n_outer
              and value_page_ids.is_contiguous(), "value_page_ids must be int32 (n_outer,) with value blocks")
        b.value_page_ids = value_page_ids.data_ptr()
    if value_shift:
        _need(value is not None and 0 < value_shift <= G, "value_shift must be in [0, G] with value blocks")
        # the shift reads rows G .. G + value_shift - 1 past each value block: they must be in its storage
        _need(min(value.stride()) >= 0, "value_shift needs non-negative value strides")
        last = value.storage_offset() + sum((n - 1) * st for n, st in zip(value.shape, value.stride())) \
            + value_shift * value.stride(-2)
        _need(last < value.untyped_storage().nbytes() // value.element_size(),
              "value_shift: rows G .. G + value_shift - 1 of a value block lie outside its tensor's storage")
        b.value_shift = int(value_shift)
    return b, dev


def quantize_into_pools(store: _hip.PageStore, key: Optional[torch.Tensor], value: Optional[torch.Tensor],
                        boost_idx: Optional[torch.Tensor], page_ids: torch.Tensor, sentinel: int,
                        value_rows: Optional[int] = None) -> None:
    """One launch over an (outer, inner=head) grid of fp16 or bf16 blocks.
    A ``cpu.PoolSet`` store (pools on the CPU) runs ``cpu.quantize_into_pools``.

    key / value: (n_outer, n_inner, G, D) fp16 or bf16 views (any strides),
    or (n_seq, n_per, n_inner, G, D) views whose n_seq * n_per blocks are
    taken sequence-major (n_outer = n_seq * n_per; a prompt's pages read in
    place); boost_idx: (n_outer, n_inner, D) or (n_inner, D) uint8;
    page_ids: (n_outer,) int32 device tensor of destination pages.
    """
    if isinstance(store, cpu.PoolSet):
        cpu.quantize_into_pools(store, key, value, boost_idx, page_ids, sentinel, value_rows)
        return
    b, dev = _quant_batch(store, key, value, boost_idx, page_ids, sentinel, value_rows)
    _hip.check(_hip.load().kitty_quantize_kv_blocks(ctypes.byref(store), ctypes.byref(b), _hip.stream_ptr(dev)))


class QuantizePlan:
    """Pre-validated arguments of one batch-quantise launch over fixed tensors
    (same arguments as :func:`quantize_into_pools`); ``run()`` only enqueues
    the kernel on the current stream.  The tensors must stay alive and in
    place while the plan is used."""

    def __init__(self, store: _hip.PageStore, key: Optional[torch.Tensor], value: Optional[torch.Tensor],
                 boost_idx: Optional[torch.Tensor], page_ids: torch.Tensor, sentinel: int,
                 value_rows: Optional[int] = None, value_page_ids: Optional[torch.Tensor] = None,
                 value_shift: int = 0) -> None:
        """value_page_ids: the value blocks' own pages (default page_ids);
        value_shift R > 0: after reading its value rows, each value block
        moves rows G .. G + R - 1 of its source to rows 0 .. R - 1 (the value
        window shift of a spill; the source's storage must hold those rows)."""
        self._b, self._dev = _quant_batch(store, key, value, boost_idx, page_ids, sentinel, value_rows,
                                          value_page_ids, value_shift)
        self._store = store
        self._keep = (key, value, boost_idx, page_ids, value_page_ids)
        self._lib = _hip.load()

    def run(self) -> None:
        _hip.check(self._lib.kitty_quantize_kv_blocks(ctypes.byref(self._store), ctypes.byref(self._b),
                                                      _hip.stream_ptr(self._dev)))


# --------------------------------------------------------------- decode

_unique_cache: "collections.OrderedDict" = collections.OrderedDict()


def boost_rows_unique(boost_idx: torch.Tensor, d_boost: int) -> bool:
    """True when no rank below d_boost repeats within a boost_idx row; the
    MFMA decode path relies on it.  Checking reads the rows back to the host
    (a device-to-host copy, which waits for the stream), so the answer is
    kept per boost tensor: keyed by its address, shape, strides and torch's
    version counter (which every in-place write through torch advances),
    with a reference that keeps the memory from being reused while the
    entry lives.  Writes that bypass torch (a kernel given the raw pointer)
    are not seen; pass ``boost_unique`` to the plan in that case."""
    t = boost_idx.detach()
    key = (t.device, t.data_ptr(), tuple(t.shape), tuple(t.stride()), t._version, int(d_boost))
    hit = _unique_cache.get(key)
    if hit is not None:
        _unique_cache.move_to_end(key)
        return hit[1]
    bi = t.to("cpu", torch.int64).reshape(-1, t.shape[-1])
    ok = True
    for row in bi:
        ranks = row[row < d_boost]
        if ranks.numel() != torch.unique(ranks).numel():
            ok = False
            break
    _unique_cache[key] = (t, ok)
    if len(_unique_cache) > 32:
        _unique_cache.popitem(last=False)
    return ok


class HostStager:
    """Small int32 host data onto the device without a blocking copy or a
    fresh pinned allocation per call: a ring of pinned staging rows,
    allocated once, and non-blocking copies on the current stream.  A row is
    rewritten only after the event recorded behind its last copy completed
    (`ring` copies earlier: in practice never a wait).  Data larger than a
    row takes a freshly pinned tensor."""

    def __init__(self, device: torch.device, cap: int, ring: int = 8) -> None:
        self.device = device
        self._buf = torch.empty(ring, cap, dtype=torch.int32, pin_memory=True)
        self._np = self._buf.numpy()
        self._ev: list = [None] * ring
        self._i = 0

    def __call__(self, a, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """`a` as an int32 device tensor (new, or the front of `out`)."""
        a = np.ascontiguousarray(a, dtype=np.int32).reshape(-1)
        n = a.size
        row = None
        if n > self._buf.shape[1]:
            src = torch.from_numpy(a).pin_memory()
        else:
            row = self._i
            self._i = (row + 1) % len(self._ev)
            if self._ev[row] is not None:
                self._ev[row].synchronize()
            self._np[row, :n] = a
            src = self._buf[row, :n]
        if out is None:
            out = src.to(self.device, non_blocking=True)
        else:
            out[:n].copy_(src, non_blocking=True)
        if row is not None:
            if self._ev[row] is None:
                self._ev[row] = torch.cuda.Event()
            self._ev[row].record()
        return out


_stagers: dict = {}


def stage_i32(values, device: torch.device) -> torch.Tensor:
    """int32 host values as a device tensor through the device's shared
    HostStager (rows of 4096 values)."""
    st = _stagers.get(device)
    if st is None:
        st = _stagers[device] = HostStager(device, 4096)
    return st(values)


class DecodePlan:
    """Validated, pre-built arguments of one batched paged-decode call.

    Building the plan does all host-side checks and allocates the workspace
    once; ``run()`` then only enqueues the kernels on the current stream, so
    a decode loop (or the benchmark) pays no Python validation per step.

    q (B, Hq, D) fp16; block_table (B, W) int32; num_pages (B,) int32;
    pools as in the layout manager; boost_idx (Hkv, D) uint8;
    sink_k/v (B, Hkv, S, D) fp16 + sink_len (B,) int32;
    tail_k/v (B, Hkv, T, D) fp16 + tail_len (B,) int32; out (B, Hq, D) fp16.
    With a bfloat16 config, q, the sinks and the tails are bfloat16 and so
    are the metadata pools; out stays fp16 (the reference returns fp16,
    kernels/attention.py:189).  ``kernel`` names the split kernel the plan
    runs ("mfma" or "generic"); a plan at the production shape that falls
    back to the generic kernel (repeated boost ranks, bf16 or misaligned
    buffers) warns once per process.

    Independent value stream (the KIVI split of the pipeline's FP16 value
    window): num_pages_v (B,) int32 value pages and tail_len_v (B,) int32
    value-tail tokens in tail_v (B, Hkv, Tv, D), with
    (num_pages - num_pages_v) * G + tail_len == tail_len_v per sequence.
    Without them both streams use num_pages and tail_len.
    """

    def __init__(self, q: torch.Tensor, block_table: torch.Tensor, num_pages: torch.Tensor,
                 key_baseline: torch.Tensor, key_boost: torch.Tensor, key_meta: torch.Tensor,
                 value_pool: torch.Tensor, value_meta: torch.Tensor, boost_idx: torch.Tensor,
                 sink_k: torch.Tensor, sink_v: torch.Tensor, sink_len: torch.Tensor,
                 tail_k: torch.Tensor, tail_v: torch.Tensor, tail_len: torch.Tensor,
                 max_pages: Optional[int] = None, pages_per_split: int = 0,
                 sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None, boost_unique: Optional[bool] = None,
                 num_pages_v: Optional[torch.Tensor] = None, tail_len_v: Optional[torch.Tensor] = None):
        dev = _hip.require_device(q, block_table, num_pages, key_baseline, key_boost, key_meta, value_pool,
                                  value_meta, boost_idx, sink_k, sink_v, sink_len, tail_k, tail_v, tail_len)
        _need((num_pages_v is None) == (tail_len_v is None), "num_pages_v and tail_len_v go together")
        B, Hq, D = q.shape
        P, Hkv, D2, G4 = key_baseline.shape
        _need(D2 == D, "head_dim mismatch between q and pools")
        act_dtype = _dtype16("q, sinks and tails", q, sink_k, sink_v, tail_k, tail_v)
        meta_dtype = _dtype16("key_metadata and value_metadata", key_meta, value_meta)
        for name, t in (("sink_k", sink_k), ("sink_v", sink_v), ("tail_k", tail_k), ("tail_v", tail_v)):
            _need(t.dim() == 4 and t.shape[0] == B and t.shape[1] == Hkv and t.shape[3] == D
                  and (t.shape[2] == 0 or t.stride(3) == 1),
                  f"{name} must be (B, Hkv, n, D) with contiguous channels")
        _need(q.stride(2) == 1, "q channels must be contiguous")
        _need(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == B
              and block_table.stride(1) == 1, "block_table must be int32 (B, W) with contiguous rows")
        lens = [("num_pages", num_pages), ("sink_len", sink_len), ("tail_len", tail_len)]
        if num_pages_v is not None:
            _hip.require_device(num_pages_v, tail_len_v)
            lens += [("num_pages_v", num_pages_v), ("tail_len_v", tail_len_v)]
        for name, t in lens:
            _need(t.dtype == torch.int32 and t.numel() == B and t.is_contiguous(), f"{name} must be int32 (B,)")
        _need(boost_idx.dtype == torch.uint8 and tuple(boost_idx.shape) == (Hkv, D) and boost_idx.is_contiguous(),
              "boost_idx must be contiguous uint8 (Hkv, D)")
        for t in (key_baseline, key_boost, key_meta, value_pool, value_meta):
            _need(t.is_contiguous(), "pools must be contiguous")
        if max_pages is None:
            max_pages = block_table.shape[1]
        _need(max_pages <= block_table.shape[1], "max_pages exceeds the block table width")
        if out is None:
            out = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
        _need(out.dtype == torch.float16 and tuple(out.shape) == (B, Hq, D) and out.stride(2) == 1, "out shape")

        a = _hip.DecodeArgs()
        a.q, a.q_s_seq, a.q_s_head = q.data_ptr(), q.stride(0), q.stride(1)
        a.out, a.out_s_seq, a.out_s_head = out.data_ptr(), out.stride(0), out.stride(1)
        a.key_low, a.key_high, a.key_meta = key_baseline.data_ptr(), key_boost.data_ptr(), key_meta.data_ptr()
        a.value, a.value_meta = value_pool.data_ptr(), value_meta.data_ptr()
        a.num_pool_pages = P
        a.block_table, a.bt_stride = block_table.data_ptr(), block_table.stride(0)
        a.num_pages, a.boost_idx = num_pages.data_ptr(), boost_idx.data_ptr()
        for name, t in (("sink_k", sink_k), ("sink_v", sink_v), ("tail_k", tail_k), ("tail_v", tail_v)):
            setattr(a, name, _hip.Fp16Seg(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2)))
        a.sink_len, a.tail_len = sink_len.data_ptr(), tail_len.data_ptr()
        a.sink_capacity, a.tail_capacity = sink_k.shape[2], tail_k.shape[2]
        _need(sink_v.shape[2] == sink_k.shape[2] and tail_v.shape[2] >= tail_k.shape[2],
              "sink_v / tail_v must hold as many tokens as sink_k / tail_k")
        if num_pages_v is not None:
            a.num_pages_v, a.tail_len_v, a.tail_v_capacity = num_pages_v.data_ptr(), tail_len_v.data_ptr(), tail_v.shape[2]
        a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim = B, Hq, Hkv, D
        a.page_tokens, a.d_boost = G4 * 4, key_boost.shape[2]
        a.max_pages, a.pages_per_split = int(max_pages), int(pages_per_split)
        if boost_unique is None:
            boost_unique = boost_rows_unique(boost_idx, key_boost.shape[2])
        a.flags = _hip.KITTY_DECODE_UNIQUE_BOOST_ROWS if boost_unique else 0
        a.sm_scale = float(1.0 / math.sqrt(D) if sm_scale is None else sm_scale)
        a.meta_dtype, a.act_dtype = meta_dtype, act_dtype
        self._L = _hip.load()
        path = ctypes.c_int32(0)
        _hip.check(self._L.kitty_decode_path(ctypes.byref(a), ctypes.byref(path)))
        self.kernel = "mfma" if path.value == _hip.KITTY_DECODE_PATH_MFMA else "generic"
        if self.kernel == "generic" and D == 128 and G4 * 4 == 128 and Hq // Hkv <= 16:
            _warn_generic(boost_unique, act_dtype, meta_dtype)
        need = ctypes.c_size_t(0)
        _hip.check(self._L.kitty_decode_workspace_size(ctypes.byref(a), ctypes.byref(need)))
        if workspace is None or workspace.numel() * workspace.element_size() < need.value:
            workspace = torch.empty(max(need.value, 16), dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        self.args = a
        self.out = out
        self.device = dev
        self._sig = ((q.device, q.dtype, q.shape, q.stride()), (out.device, out.dtype, out.shape, out.stride()))
        # keep every tensor the kernels read alive as long as the plan
        self._keep = (q, block_table, num_pages, key_baseline, key_boost, key_meta, value_pool, value_meta,
                      boost_idx, sink_k, sink_v, sink_len, tail_k, tail_v, tail_len, workspace, num_pages_v,
                      tail_len_v)

    def run(self) -> torch.Tensor:
        _hip.check(self._L.kitty_paged_decode(ctypes.byref(self.args), _hip.stream_ptr(self.device)))
        return self.out

    def run_with(self, q: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """The same decode with another query and output of the plan's
        shapes and strides (a plan cached across decode steps: everything
        else it reads is device state that the steps update in place)."""
        _need(((q.device, q.dtype, q.shape, q.stride()), (out.device, out.dtype, out.shape, out.stride())) == self._sig,
              "q and out must match the plan's dtype, shape, strides and device")
        self.args.q, self.args.out = q.data_ptr(), out.data_ptr()
        try:
            _hip.check(self._L.kitty_paged_decode(ctypes.byref(self.args), _hip.stream_ptr(self.device)))
        finally:
            self.args.q, self.args.out = self._keep[0].data_ptr(), self.out.data_ptr()
        return out

    def run_splits(self) -> None:
        _hip.check(self._L.kitty_paged_decode_splits(ctypes.byref(self.args), _hip.stream_ptr(self.device)))

    def run_merge(self) -> torch.Tensor:
        _hip.check(self._L.kitty_paged_decode_merge(ctypes.byref(self.args), _hip.stream_ptr(self.device)))
        return self.out


_warned_generic = False


def _warn_generic(boost_unique: bool, act_dtype: int, meta_dtype: int) -> None:
    global _warned_generic
    if _warned_generic:
        return
    _warned_generic = True
    if not boost_unique:
        why = "a boost_idx row repeats a rank below d_boost"
    elif act_dtype == _hip.KITTY_DTYPE_BF16 or meta_dtype == _hip.KITTY_DTYPE_BF16:
        why = "the buffers are bfloat16"
    else:
        why = "a pool or FP16 buffer is not 16-byte aligned"
    warnings.warn(f"kitty paged decode runs the shape-generic kernel because {why}; at this shape it is about "
                  "15x slower than the MFMA kernel", RuntimeWarning, stacklevel=3)


def decode_plan(*args, **kwargs):
    """``DecodePlan`` for device tensors, ``cpu.CpuDecodePlan`` (same
    arguments and methods) when q is a CPU tensor."""
    q = args[0] if args else kwargs["q"]
    if q.device.type == "cpu":
        return cpu.CpuDecodePlan(*args, **kwargs)
    return DecodePlan(*args, **kwargs)


def paged_decode(*args, **kwargs) -> torch.Tensor:
    """Batched fused paged decode attention: ``decode_plan(*args, **kwargs).run()``."""
    return decode_plan(*args, **kwargs).run()


def decode_workspace_bytes(B: int, Hq: int, Hkv: int, D: int, G: int, Dk: int, max_pages: int,
                           pages_per_split: int = 0, sink_capacity: int = 0, tail_capacity: int = 0,
                           tail_v_capacity: Optional[int] = None) -> int:
    """Workspace size for paged_decode with these shapes (for preallocation).
    The FP16 buffer capacities (tokens per (sequence, head) of sink_k, tail_k
    and, for an independent value stream, tail_v) enter the work plan, so
    pass the ones the decode will use."""
    a = _hip.DecodeArgs()
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim = B, Hq, Hkv, D
    a.page_tokens, a.d_boost, a.max_pages, a.pages_per_split = G, Dk, max_pages, pages_per_split
    a.sink_capacity, a.tail_capacity = sink_capacity, tail_capacity
    if tail_v_capacity is not None:
        a.num_pages_v = a.tail_len_v = 1  # non-null placeholders: an independent value stream
        a.tail_v_capacity = tail_v_capacity
    a.bt_stride = max(1, max_pages)
    a.block_table = a.key_low = a.key_meta = a.value = a.value_meta = a.key_high = 1  # non-null placeholders
    need = ctypes.c_size_t(0)
    _hip.check(_hip.load().kitty_decode_workspace_size(ctypes.byref(a), ctypes.byref(need)))
    return need.value
