"""CPU oracle for the quantized-KV hot path of bitxwolf/kitty-kv.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker or as the timed CPU baseline.  The product package never imports it.

Two independent restatements of the reference's PyTorch fallback live here:

* ``libkitty_oracle.so`` (``kitty_oracle.c``, built by ``oracle/Makefile``): a
  scalar C restatement, op for op, of
  ``kitty/kernels/quantize_key.py:38-124``, ``quantize_value.py:38-133``,
  ``dequantize_key.py:35-97`` and ``kitty/kernels/attention.py:46-189``.
* ``*_np`` functions below: vectorised numpy restatements of the same
  functions, written separately so that the C and numpy versions check each
  other bit for bit.

Parity pins (tests/test_oracle.py): the reference's two known-answer tests
(``tests/test_quantize.py:141-166`` and ``:247-268``), its round-trip bounds
(``:56-113``, ``:206-230``), hand-derived tie and underflow cases, brute force
over every 4-token code pattern at G=4, and the paged attention checked against
torch's ``scaled_dot_product_attention`` on the oracle's dequantised K/V.
``paged_attention_kv`` (independent key and value streams) is pinned by its
reduction to the C paged attention when both streams hold the same pages, by
the equivalence of a value page and its dequantised rows in the FP16 value
tail, and by SDPA on the assembled streams.
The bf16 helpers (``f32_to_bf16``, ``quantize_key_bf16``,
``quantize_value_bf16``; KittyConfig.dtype = "bfloat16") are pinned in
tests/test_bf16.py: the rounding equals torch's ``.to(torch.bfloat16)``, and
blocks fp16 also holds reduce to the fp16 path with bf16(fp16(x)) metadata.
Only the sign of a zero zero-point and the reference's fp32 summation order
are unpinned; both are compared by value / within tolerance.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libkitty_oracle.so")
_lib: Optional[ctypes.CDLL] = None


def build(force: bool = False) -> str:
    """Compile the C oracle with ``make`` (gcc, no fast-math, no contraction)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int
        L.kitty_oracle_quantize_key.argtypes = [P, P, I, I, I, I, P, P, P, P]
        L.kitty_oracle_quantize_value.argtypes = [P, I, I, P, P, P]
        L.kitty_oracle_dequantize_key.argtypes = [P, P, P, P, P, I, I, I, P]
        L.kitty_oracle_dequantize_value.argtypes = [P, P, P, I, I, P]
        L.kitty_oracle_paged_attention.argtypes = [
            P, P, I, P, P, P, P, P, P, I, P, P, I, P, P, I, I, I, I, I, I, P]
        L.kitty_oracle_h2f.argtypes = [ctypes.c_uint16]
        L.kitty_oracle_h2f.restype = ctypes.c_float
        L.kitty_oracle_f2h.argtypes = [ctypes.c_float]
        L.kitty_oracle_f2h.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f16bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float16)).view(np.uint16)


# --------------------------------------------------------------- C oracle

def quantize_key(key: np.ndarray, boost_idx: np.ndarray, d_boost: int, sentinel: int):
    """key (D, G) fp16 -> (t2b (D,G/4) u8, thigh (d_boost,G/4) u8, scale (D,) f16, zero (D,) f16).

    Restates ``quantize_key_page_torch`` (kitty/kernels/quantize_key.py:38-124)."""
    kb = _f16bits(key)
    D, G = kb.shape
    bi = np.ascontiguousarray(boost_idx, dtype=np.uint8)
    t2b = np.zeros((D, G // 4), np.uint8)
    thigh = np.zeros((max(d_boost, 0), G // 4), np.uint8)
    sc = np.zeros(D, np.uint16)
    zp = np.zeros(D, np.uint16)
    lib().kitty_oracle_quantize_key(_p(kb), _p(bi), D, G, d_boost, sentinel,
                                    _p(t2b), _p(thigh), _p(sc), _p(zp))
    return t2b, thigh, sc.view(np.float16), zp.view(np.float16)


def quantize_value(value: np.ndarray):
    """value (G, D) fp16 -> (packed (G, D/4) u8, scale (G,) f16, zero (G,) f16).

    Restates ``quantize_value_page_torch`` (kitty/kernels/quantize_value.py:38-90)."""
    vb = _f16bits(value)
    G, D = vb.shape
    packed = np.zeros((G, D // 4), np.uint8)
    sc = np.zeros(G, np.uint16)
    zp = np.zeros(G, np.uint16)
    lib().kitty_oracle_quantize_value(_p(vb), G, D, _p(packed), _p(sc), _p(zp))
    return packed, sc.view(np.float16), zp.view(np.float16)


def dequantize_key(t2b, thigh, scale, zero, boost_idx, d_boost: int) -> np.ndarray:
    """Restates ``dequantize_key_page_torch`` (kitty/kernels/dequantize_key.py:35-97); (D, G) fp32."""
    t2b = np.ascontiguousarray(t2b, np.uint8)
    D, G4 = t2b.shape
    thigh = np.ascontiguousarray(thigh, np.uint8)
    if thigh.size == 0:
        thigh = np.zeros((1, G4), np.uint8)
    out = np.zeros((D, G4 * 4), np.float32)
    lib().kitty_oracle_dequantize_key(_p(t2b), _p(thigh), _p(_f16bits(scale)), _p(_f16bits(zero)),
                                      _p(np.ascontiguousarray(boost_idx, np.uint8)), D, G4 * 4,
                                      d_boost, _p(out))
    return out


def dequantize_value(packed, scale, zero) -> np.ndarray:
    """Restates ``dequantize_value_page_torch`` (kitty/kernels/quantize_value.py:97-133); (G, D) fp32."""
    packed = np.ascontiguousarray(packed, np.uint8)
    G, D4 = packed.shape
    out = np.zeros((G, D4 * 4), np.float32)
    lib().kitty_oracle_dequantize_value(_p(packed), _p(_f16bits(scale)), _p(_f16bits(zero)),
                                        G, D4 * 4, _p(out))
    return out


def paged_attention(q, page_list: Sequence[int], key_baseline, key_boost, key_meta,
                    value_pool, value_meta, boost_idx, d_boost: int,
                    sink_k, sink_v, tail_k, tail_v, num_q_heads: int, num_kv_heads: int,
                    head_dim: int, n_threads: int = 0) -> np.ndarray:
    """One sequence of ``paged_attention_reference`` (kitty/kernels/attention.py:46-189).

    Pools are numpy arrays with the layout manager's shapes (layout.py:129-147);
    q (Hq, D) fp16; sinks / tails (H, n, D) fp16 (tail attended iff n > 0).
    Returns (Hq, D) fp16."""
    P, H, D, G4 = key_baseline.shape
    G = G4 * 4
    assert H == num_kv_heads and D == head_dim
    kb = np.ascontiguousarray(key_baseline, np.uint8)
    kh = np.ascontiguousarray(key_boost, np.uint8)
    if kh.size == 0:
        kh = np.zeros((1,), np.uint8)
    km = _f16bits(key_meta)
    vp = np.ascontiguousarray(value_pool, np.uint8)
    vm = _f16bits(value_meta)
    pl = np.ascontiguousarray(np.asarray(page_list, dtype=np.int32))
    if pl.size == 0:
        pl = np.zeros(1, np.int32)
    n_pages = len(page_list)
    sk, sv = _f16bits(sink_k), _f16bits(sink_v)
    tk, tv = _f16bits(tail_k), _f16bits(tail_v)
    n_sink = sk.shape[1] if sk.ndim == 3 else 0
    n_tail = tk.shape[1] if tk.ndim == 3 else 0
    if sk.size == 0:
        sk = sv = np.zeros(1, np.uint16)
    if tk.size == 0:
        tk = tv = np.zeros(1, np.uint16)
    out = np.zeros((num_q_heads, D), np.uint16)
    if n_threads <= 0:
        n_threads = min(num_kv_heads, os.cpu_count() or 1)
    lib().kitty_oracle_paged_attention(
        _p(_f16bits(q)), _p(pl), n_pages, _p(kb), _p(kh), _p(km), _p(vp), _p(vm),
        _p(np.ascontiguousarray(boost_idx, np.uint8)), d_boost,
        _p(sk), _p(sv), n_sink, _p(tk), _p(tv), n_tail,
        num_q_heads, num_kv_heads, D, G, n_threads, _p(out))
    return out.view(np.float16)


# ------------------------------------------------- numpy restatements

def _f32(x) -> np.ndarray:
    """fp16 arrays and fp32 arrays (e.g. bf16 values from bf16_to_f32) as
    fp32, exactly; any other dtype is taken as fp16 data, as the callers'
    fp16 paths always did."""
    a = np.asarray(x)
    if a.dtype == np.float32:
        return a
    return np.asarray(a, np.float16).astype(np.float32)


def quantize_key_np(key: np.ndarray, boost_idx: np.ndarray, d_boost: int, sentinel: int):
    """Vectorised numpy restatement of ``quantize_key_page_torch``
    (kitty/kernels/quantize_key.py:69-124); same outputs as :func:`quantize_key`.
    key: fp16 data, or fp32 values of bf16 data (``key.float()``, :69)."""
    x = _f32(key)
    D, G = x.shape
    boosted = np.asarray(boost_idx).astype(np.int64) < sentinel
    mn = x.min(axis=1)
    mx = x.max(axis=1)
    rng = np.maximum(mx - mn, np.float32(1e-8))
    mq = np.where(boosted, np.float32(15.0), np.float32(3.0)).astype(np.float32)
    s = (rng / mq).astype(np.float32)
    zr = np.rint(-mn / s)
    zp = np.minimum(np.where(zr > 0, zr, np.float32(0)), mq).astype(np.float32)   # -0 -> +0, as torch
    qf = np.rint(x / s[:, None]) + zp[:, None]
    c = np.minimum(np.maximum(qf, np.float32(0)), mq[:, None]).astype(np.uint8)
    lo = c & 3
    hi = (c >> 2) & 3
    t2b = np.zeros((D, G // 4), np.uint8)
    for i in range(4):
        t2b |= (lo[:, i::4] << (2 * i)).astype(np.uint8)
    thigh = np.zeros((d_boost, G // 4), np.uint8)
    bi = np.asarray(boost_idx).astype(np.int64)
    for d in np.nonzero(boosted)[0]:
        if bi[d] < d_boost:
            for i in range(4):
                thigh[bi[d]] |= (hi[d, i::4] << (2 * i)).astype(np.uint8)
    with np.errstate(over="ignore"):          # fp16 overflow gives inf, as torch's .to(float16)
        return t2b, thigh, s.astype(np.float16), zp.astype(np.float16)


def quantize_value_np(value: np.ndarray):
    """Vectorised numpy restatement of ``quantize_value_page_torch``
    (kitty/kernels/quantize_value.py:58-90); value as in quantize_key_np."""
    v = _f32(value)
    G, D = v.shape
    mn = v.min(axis=1)
    mx = v.max(axis=1)
    rng = np.maximum(mx - mn, np.float32(1e-8))
    s = (rng / np.float32(3.0)).astype(np.float32)
    zr = np.rint(-mn / s)
    zp = np.minimum(np.where(zr > 0, zr, np.float32(0)), np.float32(3)).astype(np.float32)
    c = np.minimum(np.maximum(np.rint(v / s[:, None]) + zp[:, None], np.float32(0)),
                   np.float32(3)).astype(np.uint8)
    packed = np.zeros((G, D // 4), np.uint8)
    for i in range(4):
        packed |= (c[:, i::4] << (2 * i)).astype(np.uint8)
    with np.errstate(over="ignore"):
        return packed, s.astype(np.float16), zp.astype(np.float16)


def dequantize_key_np(t2b, thigh, scale, zero, boost_idx, d_boost: int) -> np.ndarray:
    t2b = np.asarray(t2b, np.uint8)
    D, G4 = t2b.shape
    shifts = np.array([0, 2, 4, 6], np.uint8)
    lo = ((t2b[:, :, None] >> shifts) & 3).reshape(D, G4 * 4).astype(np.int32)
    hi = np.zeros_like(lo)
    bi = np.asarray(boost_idx).astype(np.int64)
    for d in range(D):
        if bi[d] < d_boost:
            hi[d] = ((np.asarray(thigh, np.uint8)[bi[d]][:, None] >> shifts) & 3).reshape(-1)
    xq = (lo | (hi << 2)).astype(np.float32)
    s = _f32(scale)[:, None]
    z = _f32(zero)[:, None]
    return ((xq - z) * s).astype(np.float32)


def dequantize_value_np(packed, scale, zero) -> np.ndarray:
    packed = np.asarray(packed, np.uint8)
    G, D4 = packed.shape
    shifts = np.array([0, 2, 4, 6], np.uint8)
    c = ((packed[:, :, None] >> shifts) & 3).reshape(G, D4 * 4).astype(np.float32)
    s = _f32(scale)[:, None]
    z = _f32(zero)[:, None]
    return ((c - z) * s).astype(np.float32)


def dequantized_kv(page_list, key_baseline, key_boost, key_meta, value_pool, value_meta,
                   boost_idx, d_boost, sink_k, sink_v, tail_k, tail_v):
    """Concatenated fp32 K, V per KV head as ``paged_attention_reference`` builds
    them (kitty/kernels/attention.py:136-168): list of (T, D) arrays per head."""
    P, H, D, G4 = key_baseline.shape
    Ks, Vs = [], []
    for h in range(H):
        kp, vp_ = [], []
        if sink_k.shape[1] > 0:
            kp.append(_f32(sink_k[h]))
            vp_.append(_f32(sink_v[h]))
        for p in page_list:
            kp.append(dequantize_key_np(key_baseline[p, h], key_boost[p, h], key_meta[p, h, 0],
                                        key_meta[p, h, 1], boost_idx[h], d_boost).T)
            vp_.append(dequantize_value_np(value_pool[p, h], value_meta[p, h, :, 0],
                                           value_meta[p, h, :, 1]))
        if tail_k.shape[1] > 0:
            kp.append(_f32(tail_k[h]))
            vp_.append(_f32(tail_v[h]))
        Ks.append(np.concatenate(kp, 0) if kp else np.zeros((0, D), np.float32))
        Vs.append(np.concatenate(vp_, 0) if vp_ else np.zeros((0, D), np.float32))
    return Ks, Vs


# ------------------------------------- independent key and value streams

def split_stream_kv(key_pages, value_pages, key_baseline, key_boost, key_meta, value_pool, value_meta,
                    boost_idx, d_boost, sink_k, sink_v, tail_k, tail_v):
    """Per KV head, the key stream sinks | key_pages | tail_k and the value
    stream sinks | value_pages | tail_v as fp32 (T, D) arrays: the layout a
    value local window gives (KIVI: keys are quantised a page at a time,
    values once they leave the last R tokens), where the most recent tokens
    of the key stream's pages may still be FP16 values.  The two streams
    must have the same length.  With value_pages == key_pages and equal
    tails this is what paged_attention_reference attends to
    (kitty/kernels/attention.py:136-168; the window's spill rule is
    kitty/pipeline.py:155-168)."""
    Ks, _ = dequantized_kv(key_pages, key_baseline, key_boost, key_meta, value_pool, value_meta,
                           boost_idx, d_boost, sink_k, sink_v, tail_k, tail_k)
    _, Vs = dequantized_kv(value_pages, key_baseline, key_boost, key_meta, value_pool, value_meta,
                           boost_idx, d_boost, sink_v, sink_v, tail_v, tail_v)
    for K, V in zip(Ks, Vs):
        if K.shape != V.shape:
            raise ValueError(f"key stream has {K.shape[0]} tokens, value stream {V.shape[0]}")
    return Ks, Vs


def paged_attention_kv(q, key_pages, value_pages, key_baseline, key_boost, key_meta, value_pool, value_meta,
                       boost_idx, d_boost: int, sink_k, sink_v, tail_k, tail_v, num_q_heads: int,
                       num_kv_heads: int, head_dim: int) -> np.ndarray:
    """(Hq, D) fp16 decode output over independent key and value streams
    (split_stream_kv): softmax(q K^T / sqrt(D)) V per query head, KV head
    qh // (Hq / H), in float64; zeros for an empty context."""
    Ks, Vs = split_stream_kv(key_pages, value_pages, key_baseline, key_boost, key_meta, value_pool, value_meta,
                             boost_idx, d_boost, sink_k, sink_v, tail_k, tail_v)
    g = num_q_heads // num_kv_heads
    out = np.zeros((num_q_heads, head_dim), np.float64)
    qd = _f32(q).astype(np.float64)
    for qh in range(num_q_heads):
        K, V = Ks[qh // g].astype(np.float64), Vs[qh // g].astype(np.float64)
        if K.shape[0] == 0:
            continue
        s = K @ qd[qh] / np.sqrt(head_dim)
        p = np.exp(s - s.max())
        out[qh] = (p / p.sum()) @ V
    return out.astype(np.float16)


# ---------------------------------------------------------------- bf16
# KittyConfig.dtype = "bfloat16" (kitty/config.py:76): buffers and metadata
# pools in bf16.  The quantisers still return fp16 scales and zero points,
# which the launchers copy into the bf16 pool views (quantize_key.py:121-122,
# 263-269; quantize_value.py:90, 223-227): a bf16 pool holds bf16(fp16(x)).
# bf16 data travels as uint16 bit patterns (numpy has no bf16 type).

def bf16_to_f32(bits) -> np.ndarray:
    """bf16 bit patterns -> fp32 values (exact)."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even, NaN -> 0x7FC0
    (torch's .to(torch.bfloat16); pinned against torch in tests)."""
    u = np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, np.uint16(0x7FC0), r).astype(np.uint16)


def meta_bf16(x_f16) -> np.ndarray:
    """An fp16 scale or zero point as a bf16 pool stores it: bf16(fp16(x))."""
    return f32_to_bf16(np.asarray(x_f16, np.float16).astype(np.float32))


def quantize_key_bf16(key_bits, boost_idx, d_boost: int, sentinel: int):
    """bf16 key block (D, G) -> (t2b, thigh, scale, zero) with scale / zero as
    the bf16 bit patterns a bf16 key_metadata pool holds."""
    t2b, thigh, s, z = quantize_key_np(bf16_to_f32(key_bits), boost_idx, d_boost, sentinel)
    return t2b, thigh, meta_bf16(s), meta_bf16(z)


def quantize_value_bf16(value_bits):
    """bf16 value block (G, D) -> (packed, scale, zero), scale / zero as bf16 bits."""
    packed, s, z = quantize_value_np(bf16_to_f32(value_bits))
    return packed, meta_bf16(s), meta_bf16(z)
