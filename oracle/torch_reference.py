"""Op-for-op torch (CPU) restatement of the reference's paged decode path
and of its page quantisers.

TEST INFRASTRUCTURE ONLY: timed as the CPU baseline by bench.py and checked
against the C oracle by tests/test_oracle.py.  The product never imports it.

It performs the same tensor operations, in the same order and with the
same per-element Python work, as the reference's CPU path, so its time is
what a reference user pays on this host:

* ``dequantize_key_page`` follows ``kitty/kernels/dequantize_key.py:35-97``:
  a shift-and-mask unpack of the low bits of every channel, then one Python
  iteration per channel, with a ``.item()`` for each boosted one, for the high
  bits, and ``(x - zero) * scale`` in fp32.
* ``dequantize_value_page`` follows ``kitty/kernels/quantize_value.py:97-133``.
* ``quantize_key_page`` follows ``kitty/kernels/quantize_key.py:38-124``: fp32
  per-channel min / max, range clamped to 1e-8, INT4 or INT2 per channel,
  rounded codes, four codes per byte, then one Python iteration with an
  ``.item()`` per boosted channel for the high bits; ``quantize_value_page``
  follows ``kitty/kernels/quantize_value.py:38-90`` (per token, INT2).
* ``paged_attention`` follows ``kitty/kernels/attention.py:46-189``: the first
  pass over every (page, head), whose dequantised blocks are thrown away
  (lines 100-132), the per-head rebuild of K and V from sinks, pages and
  buffer tokens (lines 134-164), and per query head a score vector, softmax
  and weighted sum (lines 166-189).
"""
from __future__ import annotations

import math
from typing import List, Sequence

import torch

_SHIFTS = (0, 2, 4, 6)


def _unpack2(packed: torch.Tensor) -> torch.Tensor:
    """(R, C) uint8 of four 2-bit codes per byte (token / channel 4j + a in
    bits 2a, 2a + 1) -> (R, 4C) int32."""
    shifts = torch.tensor(_SHIFTS, dtype=torch.uint8)
    codes = (packed.unsqueeze(-1) >> shifts) & 0x03
    return codes.to(torch.int32).reshape(packed.shape[0], packed.shape[1] * 4)


def dequantize_key_page(t2b: torch.Tensor, thigh: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor,
                        boost_idx: torch.Tensor, d_boost: int) -> torch.Tensor:
    """(D, G/4) low bits, (D_boost, G/4) high bits, (D,) fp16 scale / zero,
    (D,) uint8 ranks -> (D, G) fp32 (dequantize_key.py:35-97)."""
    D = t2b.shape[0]
    low = _unpack2(t2b)
    high = torch.zeros_like(low)
    ranks = boost_idx.to(torch.int32)
    boosted = ranks < d_boost
    for d in range(D):                       # one Python step per channel, as the reference
        if boosted[d]:
            r = int(ranks[d].item())
            high[d] = _unpack2(thigh[r:r + 1])[0]
    q = (low | (high << 2)).float()
    return (q - zero.float().unsqueeze(1)) * scale.float().unsqueeze(1)


def dequantize_value_page(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor) -> torch.Tensor:
    """(G, D/4) codes, (G,) fp16 scale / zero -> (G, D) fp32
    (quantize_value.py:97-133)."""
    q = _unpack2(packed).float()
    return (q - zero.float().unsqueeze(1)) * scale.float().unsqueeze(1)


def _page_kv(h: int, pid: int, key_baseline, key_boost, key_meta, value_pool, value_meta, boost_idx,
             d_boost: int):
    k = dequantize_key_page(key_baseline[pid, h], key_boost[pid, h], key_meta[pid, h, 0], key_meta[pid, h, 1],
                            boost_idx[h], d_boost)
    v = dequantize_value_page(value_pool[pid, h], value_meta[pid, h, :, 0], value_meta[pid, h, :, 1])
    return k.T.float(), v.float()


def paged_attention(q: torch.Tensor, page_list: Sequence[int], key_baseline: torch.Tensor,
                    key_boost: torch.Tensor, key_meta: torch.Tensor, value_pool: torch.Tensor,
                    value_meta: torch.Tensor, boost_idx: torch.Tensor, d_boost: int, sink_k: torch.Tensor,
                    sink_v: torch.Tensor, buf_k: torch.Tensor, buf_v: torch.Tensor, num_q_heads: int,
                    num_kv_heads: int, head_dim: int) -> torch.Tensor:
    """(Hq, D) fp16 output of one decode step over sinks | pages | buffer
    tokens, all CPU tensors in the reference's pool layouts
    (attention.py:46-189)."""
    pages = [int(p) for p in page_list]
    kv = (key_baseline, key_boost, key_meta, value_pool, value_meta, boost_idx, d_boost)
    # first pass (attention.py:100-132): every (page, head) dequantised, results dropped
    first_k: List[torch.Tensor] = []
    for pid in pages:
        for h in range(num_kv_heads):
            k, v = _page_kv(h, pid, *kv)
            if h == 0 and len(first_k) <= len(pages):
                first_k.append(k.unsqueeze(0))
    del first_k
    # per-head K / V (attention.py:134-164)
    keys, vals = [], []
    for h in range(num_kv_heads):
        kp, vp = [], []
        if sink_k.shape[1] > 0:
            kp.append(sink_k[h].float())
            vp.append(sink_v[h].float())
        for pid in pages:
            k, v = _page_kv(h, pid, *kv)
            kp.append(k)
            vp.append(v)
        if buf_k.shape[1] > 0:
            kp.append(buf_k[h].float())
            vp.append(buf_v[h].float())
        keys.append(torch.cat(kp, 0) if kp else torch.zeros(0, head_dim))
        vals.append(torch.cat(vp, 0) if vp else torch.zeros(0, head_dim))
    # per query head (attention.py:166-189)
    group = num_q_heads // num_kv_heads
    scale = 1.0 / math.sqrt(head_dim)
    qf = q.float()
    rows = []
    for qh in range(num_q_heads):
        K, V = keys[qh // group], vals[qh // group]
        if K.shape[0] == 0:
            rows.append(torch.zeros(head_dim))
            continue
        w = torch.softmax((qf[qh] @ K.T) * scale, dim=0)
        rows.append((w.unsqueeze(1) * V).sum(dim=0))
    return torch.stack(rows, 0).to(torch.float16)


def _pack4(codes: torch.Tensor) -> torch.Tensor:
    """Four 2-bit codes per byte along the last dimension, code i of a group
    in bits 2i (quantize_key.py:106-110, quantize_value.py:85-88)."""
    out = torch.zeros(*codes.shape[:-1], codes.shape[-1] // 4, dtype=torch.uint8)
    for i in range(4):
        out |= (codes[..., i::4] << (2 * i)).to(torch.uint8)
    return out


def quantize_key_page(key: torch.Tensor, boost_idx: torch.Tensor, d_boost: int, sentinel: int):
    """key (D, G) fp16 -> (low codes (D, G/4), high codes (d_boost, G/4) u8,
    scale (D,) fp16, zero point (D,) fp16), quantize_key.py:69-124."""
    x = key.float()
    D, G = x.shape
    boosted = boost_idx < sentinel
    lo, hi = x.min(dim=1).values, x.max(dim=1).values
    mq = torch.where(boosted, torch.tensor(15.0), torch.tensor(3.0))
    s = (hi - lo).clamp(min=1e-8) / mq
    z = torch.minimum(torch.maximum((-lo / s).round(), torch.zeros_like(s)), mq)
    qf = (x / s[:, None]).round() + z[:, None]
    q = torch.minimum(torch.maximum(qf, torch.zeros_like(qf)), mq[:, None]).to(torch.uint8)
    low = _pack4(q & 3)
    high = torch.zeros(d_boost, G // 4, dtype=torch.uint8)
    hq = (q >> 2) & 3
    for d in torch.where(boosted)[0]:
        r = int(boost_idx[d].item())
        if r < d_boost:
            for i in range(4):
                high[r] |= (hq[d, i::4] << (2 * i)).to(torch.uint8)
    return low, high, s.to(torch.float16), z.to(torch.float16)


def quantize_value_page(value: torch.Tensor):
    """value (G, D) fp16 -> (codes (G, D/4) u8, scale (G,) fp16, zero point
    (G,) fp16), quantize_value.py:58-90."""
    x = value.float()
    lo, hi = x.min(dim=1).values, x.max(dim=1).values
    s = (hi - lo).clamp(min=1e-8) / 3.0
    three = torch.full_like(s, 3.0)
    z = torch.minimum(torch.maximum((-lo / s).round(), torch.zeros_like(s)), three)
    qf = (x / s[:, None]).round() + z[:, None]
    q = torch.minimum(torch.maximum(qf, torch.zeros_like(qf)), torch.full_like(qf, 3.0)).to(torch.uint8)
    return _pack4(q), s.to(torch.float16), z.to(torch.float16)
