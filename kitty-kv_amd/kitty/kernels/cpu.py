"""The kitty.kernels functions for CPU tensors.

The reference runs every kernel function on CPU tensors through its PyTorch
code (``kernels/attention.py:46-50, 320-341``, ``quantize_key.py:245-269``,
``quantize_value.py:197-227``, ``dequantize_key.py:169-228``), and its
config-1 plumbing case is a CPU decode step.  This module gives the package
the same ability with vectorised torch code: every block of a batch, every
page and head of a sequence in a few tensor operations, no Python loop per
channel, page or head.

* Quantisation keeps the reference's fp32 operation order (min / max, range
  clamped to 1e-8, ``s = range / mq``, ``z = clamp(round(-min / s), 0, mq)``,
  ``c = clamp(round(x / s) + z, 0, mq)``, half-to-even rounding, fp16 scale
  and zero point), so codes, scales and zero points are bit-identical to the
  reference's and to the HIP kernels'.
* Dequantisation is ``(code - z) * s`` in fp32 from the stored metadata.
* Decode is softmax attention in fp32 over sinks, dequantised pages and the
  FP16 tails, with the GQA map ``kv head = q head // (Hq / Hkv)``
  (``kernels/attention.py:166-189``), batched over the query heads of each KV
  head; the key and value streams may hold different page counts (the
  pipeline's value window).

Dispatch is by device only: the callers send CPU tensors here and ROCm
device tensors to libkitty_hip.so.  A device tensor is never computed here
(those wrappers raise when the library is missing).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

_SHIFTS = torch.tensor([0, 2, 4, 6], dtype=torch.uint8)


def _unpack2(packed: torch.Tensor) -> torch.Tensor:
    """(..., n) uint8 holding four 2-bit codes per byte (element 4j + a in
    bits 2a, 2a + 1 of byte j) -> (..., 4n) uint8 codes."""
    return ((packed.unsqueeze(-1) >> _SHIFTS) & 3).flatten(-2)


def _pack2(codes: torch.Tensor) -> torch.Tensor:
    """(..., 4n) uint8 codes in 0..3 -> (..., n) uint8, element 4j + a in bits
    2a, 2a + 1 of byte j (quantize_key.py:102-110, quantize_value.py:78-88)."""
    c = codes.unflatten(-1, (-1, 4))
    return c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)


def _clamp_round(x: torch.Tensor, lo: torch.Tensor, hi: torch.Tensor) -> torch.Tensor:
    """min(max(x, lo), hi), the reference's element-wise clamp (the sign of a
    zero result is torch's, as in quantize_key.py:87, 97-99)."""
    return torch.minimum(torch.maximum(x, lo), hi)


# ------------------------------------------------------------- quantise

def quantize_key_blocks(key: torch.Tensor, boost_idx: torch.Tensor, d_boost: int,
                        sentinel: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Channel-major key blocks (..., D, G) (fp16, bf16 or fp32) and their
    boost_idx rows (..., D) uint8 (broadcast over the leading dimensions) ->
    Tensor_2bits (..., D, G/4) uint8, Tensor_High_2bits (..., d_boost, G/4)
    uint8, scale (..., D) fp16, zero point (..., D) fp16, each block as
    quantize_key.py:38-124 computes it.  Boosted channels (boost_idx <
    sentinel) take INT4 codes; the high 2 bits of a channel with rank
    r < d_boost go to row r, OR-ed when ranks repeat; rows no channel
    names are 0."""
    x = key.float()
    D, G = x.shape[-2:]
    if G % 4:
        raise AssertionError("G must be divisible by 4 for uint8 packing")
    bi = boost_idx.to(torch.int64).expand(*x.shape[:-2], D)
    mn = x.amin(-1)
    mx = x.amax(-1)
    rng = (mx - mn).clamp(min=1e-8)
    mq = torch.full_like(rng, 3.0).masked_fill_(bi < sentinel, 15.0)
    s = rng / mq
    zero = torch.zeros_like(rng)
    zp = _clamp_round((-mn / s).round(), zero, mq)
    c = _clamp_round((x / s.unsqueeze(-1)).round() + zp.unsqueeze(-1), zero.unsqueeze(-1),
                     mq.unsqueeze(-1)).to(torch.uint8)
    t2b = _pack2(c & 3)
    hi = (c >> 2) & 3
    # high rows: OR over the channels of each rank, one bit plane at a time
    # (amax of 0/1 values is their OR); channels without a high row go to a
    # spare row d_boost that is dropped
    rows = torch.where(bi < d_boost, bi, torch.full_like(bi, d_boost))
    planes = torch.stack((hi & 1, hi >> 1), -1)                              # (..., D, G, 2)
    acc = torch.zeros(*x.shape[:-2], d_boost + 1, G, 2, dtype=torch.uint8)
    acc.scatter_reduce_(-3, rows[..., None, None].expand(planes.shape), planes, reduce="amax")
    thigh = _pack2(acc[..., :d_boost, :, 0] | (acc[..., :d_boost, :, 1] << 1))
    return t2b, thigh, s.to(torch.float16), zp.to(torch.float16)


def quantize_value_blocks(value: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Token-major value blocks (..., G, D) -> packed (..., G, D/4) uint8,
    scale (..., G) fp16, zero point (..., G) fp16: per-token INT2 as
    quantize_value.py:38-90 computes it.  A constant token stores scale 0
    (1e-8 / 3 in fp16) and codes 3 (positive) or 0."""
    v = value.float()
    if v.shape[-1] % 4:
        raise AssertionError("head_dim D must be divisible by 4 for packing")
    mn = v.amin(-1)
    mx = v.amax(-1)
    s = (mx - mn).clamp(min=1e-8) / 3.0
    zero, three = torch.zeros_like(s), torch.full_like(s, 3.0)
    zp = _clamp_round((-mn / s).round(), zero, three)
    c = _clamp_round((v / s.unsqueeze(-1)).round() + zp.unsqueeze(-1), zero.unsqueeze(-1),
                     three.unsqueeze(-1)).to(torch.uint8)
    return _pack2(c), s.to(torch.float16), zp.to(torch.float16)


# ----------------------------------------------------------- dequantise

def dequantize_key_blocks(t2b: torch.Tensor, thigh: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor,
                          boost_idx: torch.Tensor, d_boost: int) -> torch.Tensor:
    """(..., D, G) float32 keys of packed blocks (dequantize_key.py:35-97):
    code = low | high << 2 with the high bits from row boost_idx[d] when
    boost_idx[d] < d_boost, then (code - z) * s in fp32."""
    code = _unpack2(t2b)                                                   # (..., D, G)
    if d_boost > 0:
        bi = boost_idx.to(torch.int64).expand(code.shape[:-1])
        has = bi < d_boost
        hi_rows = _unpack2(thigh)                                          # (..., d_boost, G)
        hi_rows = hi_rows.expand(*code.shape[:-2], *hi_rows.shape[-2:])
        hi = torch.gather(hi_rows, -2, bi.clamp(max=d_boost - 1).unsqueeze(-1).expand(code.shape))
        code = code | ((hi * has.unsqueeze(-1).to(torch.uint8)) << 2)
    return (code.float() - zero.float().unsqueeze(-1)) * scale.float().unsqueeze(-1)


def dequantize_value_blocks(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor) -> torch.Tensor:
    """(..., G, D) float32 values: (code - z_t) * s_t (quantize_value.py:97-133)."""
    return (_unpack2(packed).float() - zero.float().unsqueeze(-1)) * scale.float().unsqueeze(-1)


# --------------------------------------------------------------- pools

class PoolSet:
    """The five pools of a layout manager on the CPU: where the pipeline's
    spills write (the CPU counterpart of the device page store)."""

    def __init__(self, key_baseline: torch.Tensor, key_boost: torch.Tensor, key_meta: torch.Tensor,
                 value_pool: torch.Tensor, value_meta: torch.Tensor) -> None:
        self.key_baseline, self.key_boost, self.key_meta = key_baseline, key_boost, key_meta
        self.value_pool, self.value_meta = value_pool, value_meta
        self.num_pages, self.num_kv_heads, self.head_dim = key_baseline.shape[:3]
        self.page_tokens = key_baseline.shape[3] * 4
        self.d_boost = key_boost.shape[2]


def _blocks(x: torch.Tensor) -> torch.Tensor:
    """(n, H, G, D) or (n_seq, n_per, H, G, D) blocks -> (n, H, G, D), the
    second taken sequence-major."""
    return x.flatten(0, 1) if x.dim() == 5 else x


def quantize_into_pools(pools: PoolSet, key: Optional[torch.Tensor], value: Optional[torch.Tensor],
                        boost_idx: Optional[torch.Tensor], page_ids: torch.Tensor, sentinel: int,
                        value_rows: Optional[int] = None) -> None:
    """quantize_into_pools for CPU tensors: block i of key / value (n, H, G, D)
    token-major (or (n_seq, n_per, H, G, D)) into every head of page
    page_ids[i]; boost_idx (n, H, D) or (H, D).  Value rows at or past
    value_rows are quantised as zeros (pipeline.py:240-243); blocks whose page
    id lies outside the pool are not written, as on the device."""
    ids = page_ids.to(torch.int64).reshape(-1)
    ok = (ids >= 0) & (ids < pools.num_pages)
    sel = ok.nonzero().reshape(-1)
    pages = ids[sel]
    if key is not None:
        kb = _blocks(key).index_select(0, sel).transpose(-1, -2)           # (n, H, D, G)
        bi = boost_idx if boost_idx.dim() == 2 else boost_idx.index_select(0, sel)
        t2b, th, s, z = quantize_key_blocks(kb, bi, pools.d_boost, sentinel)
        dt = pools.key_meta.dtype
        pools.key_baseline[pages] = t2b
        pools.key_boost[pages] = th
        pools.key_meta[pages] = torch.stack((s.to(dt), z.to(dt)), 2)
    if value is not None:
        vb = _blocks(value).index_select(0, sel)                           # (n, H, G, D)
        if value_rows is not None and value_rows < vb.shape[2]:
            vb = vb.clone()
            vb[:, :, max(0, int(value_rows)):] = 0
        packed, s, z = quantize_value_blocks(vb)
        dt = pools.value_meta.dtype
        pools.value_pool[pages] = packed
        pools.value_meta[pages] = torch.stack((s.to(dt), z.to(dt)), -1)


# -------------------------------------------------------------- decode

def attend(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, sm_scale: float) -> torch.Tensor:
    """Softmax attention of q (Hq, D) over keys / values (Hkv, T, D), query
    head h on KV head h // (Hq / Hkv) (kernels/attention.py:166-189): fp32
    (Hq, D); zeros when T = 0."""
    Hq, D = q.shape
    Hkv, T = keys.shape[:2]
    if T == 0:
        return torch.zeros(Hq, D, dtype=torch.float32)
    qg = q.float().reshape(Hkv, Hq // Hkv, D)
    w = torch.softmax(torch.matmul(qg, keys.transpose(1, 2)) * sm_scale, dim=-1)
    return torch.matmul(w, values).reshape(Hq, D)


def _page_kv(pools: PoolSet, boost_idx: torch.Tensor, d_boost: int, kpages: torch.Tensor,
             vpages: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dequantised keys of kpages and values of vpages, (H, n G, D) fp32 each."""
    H, D = boost_idx.shape
    G = pools.page_tokens
    k = dequantize_key_blocks(pools.key_baseline[kpages], pools.key_boost[kpages], pools.key_meta[kpages, :, 0],
                              pools.key_meta[kpages, :, 1], boost_idx, d_boost)        # (n, H, D, G)
    v = dequantize_value_blocks(pools.value_pool[vpages], pools.value_meta[vpages, :, :, 0],
                                pools.value_meta[vpages, :, :, 1])                     # (n, H, G, D)
    return (k.permute(1, 0, 3, 2).reshape(H, kpages.numel() * G, D),
            v.transpose(0, 1).reshape(H, vpages.numel() * G, D))


class CpuDecodePlan:
    """Batched paged decode on CPU tensors with the arguments and methods of
    ``kernels.ops.DecodePlan``: q (B, Hq, D), block_table (B, W) int32,
    num_pages (B,), the five pools, boost_idx (Hkv, D), sink_k / sink_v
    (B, Hkv, S, D) with sink_len, tail_k (B, Hkv, T, D) with tail_len,
    tail_v (B, Hkv, Tv, D), and optionally num_pages_v / tail_len_v for an
    independent value stream.  Lengths and buffers are read when the plan
    runs, so a plan over the pipeline's views serves every later step.  A
    sequence whose lengths are inconsistent or whose page ids lie outside the
    pool gets a NaN output, as on the device."""

    kernel = "cpu"

    def __init__(self, q: torch.Tensor, block_table: torch.Tensor, num_pages: torch.Tensor,
                 key_baseline: torch.Tensor, key_boost: torch.Tensor, key_meta: torch.Tensor,
                 value_pool: torch.Tensor, value_meta: torch.Tensor, boost_idx: torch.Tensor,
                 sink_k: torch.Tensor, sink_v: torch.Tensor, sink_len: torch.Tensor,
                 tail_k: torch.Tensor, tail_v: torch.Tensor, tail_len: torch.Tensor,
                 max_pages: Optional[int] = None, pages_per_split: int = 0,
                 sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None, boost_unique: Optional[bool] = None,
                 num_pages_v: Optional[torch.Tensor] = None, tail_len_v: Optional[torch.Tensor] = None):
        tensors = (q, block_table, num_pages, key_baseline, key_boost, key_meta, value_pool, value_meta, boost_idx,
                   sink_k, sink_v, sink_len, tail_k, tail_v, tail_len, num_pages_v, tail_len_v)
        if any(t is not None and t.device.type != "cpu" for t in tensors):
            raise RuntimeError("CpuDecodePlan takes CPU tensors only")
        if (num_pages_v is None) != (tail_len_v is None):
            raise ValueError("num_pages_v and tail_len_v go together")
        B, Hq, D = q.shape
        Hkv = key_baseline.shape[1]
        if Hq % Hkv or boost_idx.shape != (Hkv, D) or key_baseline.shape[2] != D:
            raise ValueError("q, pools and boost_idx shapes do not match")
        self.pools = PoolSet(key_baseline, key_boost, key_meta, value_pool, value_meta)
        self.boost_idx = boost_idx
        self.block_table, self.num_pages, self.num_pages_v = block_table, num_pages, num_pages_v
        self.sinks = (sink_k, sink_v, sink_len)
        self.tails = (tail_k, tail_v, tail_len, tail_len_v)
        self.max_pages = block_table.shape[1] if max_pages is None else int(max_pages)
        self.sm_scale = float(1.0 / math.sqrt(D) if sm_scale is None else sm_scale)
        self.q = q
        self.out = torch.empty(B, Hq, D, dtype=torch.float16) if out is None else out
        self.device = q.device

    def _sequence(self, b: int, q: torch.Tensor) -> torch.Tensor:
        P, G = self.pools.num_pages, self.pools.page_tokens
        sink_k, sink_v, sink_len = self.sinks
        tail_k, tail_v, tail_len, tail_len_v = self.tails
        npk = int(self.num_pages[b])
        npv = npk if self.num_pages_v is None else int(self.num_pages_v[b])
        ns, nt = int(sink_len[b]), int(tail_len[b])
        ntv = nt if tail_len_v is None else int(tail_len_v[b])
        bad = not (0 <= npv <= npk <= self.max_pages and 0 <= ns <= sink_k.shape[2] and 0 <= nt <= tail_k.shape[2]
                   and 0 <= ntv <= tail_v.shape[2] and (npk - npv) * G + nt == ntv)
        pages = self.block_table[b, :npk].to(torch.int64) if not bad else None
        if bad or bool(((pages < 0) | (pages >= P)).any()):
            return torch.full(q.shape, float("nan"))
        kp, vp = _page_kv(self.pools, self.boost_idx, self.pools.d_boost, pages, pages[:npv])
        keys = torch.cat((sink_k[b, :, :ns].float(), kp, tail_k[b, :, :nt].float()), 1)
        values = torch.cat((sink_v[b, :, :ns].float(), vp, tail_v[b, :, :ntv].float()), 1)
        return attend(q, keys, values, self.sm_scale)

    def run_with(self, q: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        if q.shape != self.q.shape or out.shape != self.out.shape:
            raise ValueError("q and out must match the plan's shapes")
        for b in range(q.shape[0]):
            out[b] = self._sequence(b, q[b]).to(out.dtype)
        return out

    def run(self) -> torch.Tensor:
        return self.run_with(self.q, self.out)

    def run_splits(self) -> None:
        self.run()

    def run_merge(self) -> torch.Tensor:
        return self.out


def paged_attention(q: torch.Tensor, page_list, key_baseline: torch.Tensor, key_boost: torch.Tensor,
                    key_meta: torch.Tensor, value_pool: torch.Tensor, value_meta: torch.Tensor,
                    boost_idx: torch.Tensor, D_boost: int, sink_k: torch.Tensor, sink_v: torch.Tensor,
                    qbuf_k: torch.Tensor, qbuf_v: torch.Tensor, num_q_heads: int, num_kv_heads: int,
                    head_dim: int) -> torch.Tensor:
    """The reference-signature decode (kernels/attention.py:46-189) on CPU
    tensors: sinks, then every page of page_list, then the tail, which is
    attended only when qbuf_k holds tokens; (num_q_heads, head_dim) fp16."""
    pools = PoolSet(key_baseline, key_boost, key_meta, value_pool, value_meta)
    pages = torch.tensor(list(page_list), dtype=torch.int64)
    kp, vp = _page_kv(pools, boost_idx, D_boost, pages, pages)
    ks, vs = [sink_k.float()], [sink_v.float()]
    if qbuf_k.shape[1] > 0:
        kt, vt = [qbuf_k.float()], [qbuf_v.float()]
    else:
        kt, vt = [], []
    keys = torch.cat(ks + [kp] + kt, 1)
    values = torch.cat(vs + [vp] + vt, 1)
    return attend(q, keys, values, 1.0 / math.sqrt(head_dim)).to(torch.float16)
