"""Pins of the CPU oracle (oracle/) — the checker every GPU parity test uses.

Each check is chosen so that a plausible mistake in the restatement fails it:
* the reference's own known-answer tests (tests/test_quantize.py:141-166, :247-268);
* grid-aligned brute force: every 4-token pattern that spans the full code range
  must be reproduced exactly (catches a wrong sign/offset of the zero point, a
  transposed packing order, a wrong bit position);
* round-half-to-even ties (torch.round) vs round-half-away;
* codes from the fp32 scale, not the stored fp16 scale (quantize_key.py:84,95,121);
* fp16 underflow of the scale for constant / all-zero rows;
* the reference's round-trip error bounds (tests/test_quantize.py:56-113, :206-230);
* C restatement == independent numpy restatement, bit for bit, on random data;
* paged attention == torch scaled_dot_product_attention (float64) on the
  dequantised K/V (kitty/kernels/attention.py:136-189 is textbook attention).
"""
from fractions import Fraction
import itertools

import numpy as np
import pytest
import torch

import oracle as O


def _boost(D, d_boost, sentinel, channels=None):
    bi = np.full(D, sentinel, np.uint8)
    chans = range(d_boost) if channels is None else channels
    for r, c in enumerate(chans):
        bi[c] = r
    return bi


def test_known_answer_key_packing():
    # tests/test_quantize.py:141-166: per channel [0,1,2,3] -> scale 1, zp 0, exact.
    key = np.tile(np.array([0, 1, 2, 3], np.float16), (4, 1))
    t2b, thigh, s, z = O.quantize_key(key, np.full(4, 255, np.uint8), 0, 255)
    assert (t2b == 0xE4).all()                       # token 4j+i at bits 2i
    assert (s.astype(np.float32) == 1.0).all() and (z.astype(np.float32) == 0.0).all()
    recon = O.dequantize_key(t2b, thigh, s, z, np.full(4, 255, np.uint8), 0)
    assert np.array_equal(recon, np.tile(np.array([0, 1, 2, 3], np.float32), (4, 1)))


def test_known_answer_constant_value():
    # tests/test_quantize.py:247-268: constant 3.0 -> equal reconstruction; by
    # the formula the scale underflows to fp16 0 and every code is 3.
    v = np.full((8, 16), 3.0, np.float16)
    p, s, z = O.quantize_value(v)
    assert (p == 0xFF).all()
    assert (s.astype(np.float32) == 0).all() and (z.astype(np.float32) == 0).all()
    assert (O.dequantize_value(p, s, z) == 0).all()


def test_all_zero_blocks():
    k = np.zeros((8, 8), np.float16)
    t2b, thigh, s, z = O.quantize_key(k, _boost(8, 2, 3), 2, 3)
    assert (t2b == 0).all() and (thigh == 0).all() and (s.astype(np.float32) == 0).all()
    p, s, z = O.quantize_value(k)
    assert (p == 0).all() and (s.astype(np.float32) == 0).all()


@pytest.mark.parametrize("mq,boosted", [(3, False), (15, True)])
def test_grid_aligned_brute_force(mq, boosted):
    """Every 4-token code pattern containing 0 and mq, placed on a grid of step
    k with offset z0, must quantise to exactly those codes (s = k, z = z0)."""
    D, G = 1, 4
    sentinel = 2
    bi = np.array([0 if boosted else sentinel], np.uint8)
    levels = range(mq + 1) if mq == 3 else (0, 1, 7, 14, 15)
    n = 0
    for codes in itertools.product(levels, repeat=4):
        if 0 not in codes or mq not in codes:
            continue
        for k, z0 in ((1.0, 0), (0.25, 1), (2.0, mq)):
            x = np.array([[(c - z0) * k for c in codes]], np.float16)
            t2b, thigh, s, z = O.quantize_key(x, bi, 1, sentinel)
            assert float(s[0]) == k and float(z[0]) == z0
            lo = [(t2b[0, 0] >> (2 * i)) & 3 for i in range(4)]
            hi = [(thigh[0, 0] >> (2 * i)) & 3 for i in range(4)] if boosted else [0] * 4
            assert [l | (h << 2) for l, h in zip(lo, hi)] == list(codes)
            n += 1
            if not boosted:  # the value quantiser is the same arithmetic along D
                p, sv, zv = O.quantize_value(x.reshape(1, 4))
                assert [(p[0, 0] >> (2 * i)) & 3 for i in range(4)] == list(codes)
    assert n > 0


def test_round_half_to_even():
    # s = 1, z = 0; 0.5 -> 0, 2.5 -> 2 under half-even (half-away would give 1, 3).
    x = np.array([[0.0, 3.0, 0.5, 2.5]], np.float16)
    t2b, _, s, z = O.quantize_key(x, np.array([9], np.uint8), 0, 9)
    assert [(t2b[0, 0] >> (2 * i)) & 3 for i in range(4)] == [0, 3, 0, 2]
    # zero point tie: min = -1.5, s = 1 -> z = rint(1.5) = 2
    x = np.array([[-1.5, 1.5, 0.0, 0.0]], np.float16)
    _, _, s, z = O.quantize_key(x, np.array([9], np.uint8), 0, 9)
    assert float(s[0]) == 1.0 and float(z[0]) == 2.0


def _round_half_even(fr: Fraction) -> int:
    f = fr.numerator // fr.denominator
    rem = fr - f
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and f % 2 == 1):
        return f + 1
    return f


def test_codes_use_fp32_scale():
    """Find a channel whose code differs between the fp32 scale and its fp16
    rounding, and check the oracle follows the fp32 scale (quantize_key.py:84,95),
    with the expected code computed in exact rational arithmetic."""
    rng = np.random.default_rng(7)
    found = 0
    for _ in range(20000):
        x = rng.standard_normal(4).astype(np.float16)
        xf = x.astype(np.float32)
        rngv = np.float32(xf.max() - xf.min())
        s32 = np.float32(rngv / np.float32(3.0))
        s16 = np.float32(np.float16(s32))
        zf = np.float32(np.rint(np.float32(-xf.min()) / s32))
        z = min(max(zf, 0.0), 3.0)
        for t in range(4):
            a = min(max(_round_half_even(Fraction(float(np.float32(xf[t] / s32)))) + int(z), 0), 3)
            b = min(max(_round_half_even(Fraction(float(np.float32(xf[t] / s16)))) + int(z), 0), 3)
            if a != b:
                t2b, _, s, _ = O.quantize_key(x.reshape(1, 4), np.array([9], np.uint8), 0, 9)
                assert (t2b[0, 0] >> (2 * t)) & 3 == a
                found += 1
                break
        if found >= 5:
            break
    assert found >= 1


def test_reference_round_trip_bounds():
    rng = np.random.default_rng(1)
    D, G = 16, 8
    for _ in range(20):
        # tests/test_quantize.py:56-84 INT2 < 0.35 * range
        k = rng.standard_normal((D, G)).astype(np.float16)
        bi = np.full(D, 5, np.uint8)
        r = O.dequantize_key(*O.quantize_key(k, bi, 4, 5), bi, 4)
        assert np.abs(k.astype(np.float32) - r).max() < 0.35 * float(k.max() - k.min())
        # :86-113 INT4 (15/16 boosted) < 0.12 * range of the boosted rows
        bi = _boost(D, 15, 16)
        r = O.dequantize_key(*O.quantize_key(k, bi, 15, 16), bi, 15)
        kb = k[:15].astype(np.float32)
        assert np.abs(kb - r[:15]).max() < 0.12 * float(kb.max() - kb.min())
        # :206-230 values < 0.35 * per-token range + 1e-3
        v = rng.standard_normal((G, D)).astype(np.float16)
        rv = O.dequantize_value(*O.quantize_value(v))
        vf = v.astype(np.float32)
        assert (np.abs(vf - rv).max(1) < 0.35 * (vf.max(1) - vf.min(1)) + 1e-3).all()


def test_half_step_bound_and_extremes():
    """Unclamped elements reconstruct within half a step; the channel minimum
    maps to code 0 whenever the zero point is not clamped."""
    rng = np.random.default_rng(2)
    k = (rng.standard_normal((64, 32)) * 3).astype(np.float16)
    bi = _boost(64, 8, 9, channels=rng.permutation(64)[:8])
    t2b, th, s, z = O.quantize_key(k, bi, 8, 9)
    r = O.dequantize_key(t2b, th, s, z, bi, 8)
    kf = k.astype(np.float32)
    s32 = np.maximum(kf.max(1) - kf.min(1), np.float32(1e-8)) / np.where(bi < 9, 15, 3).astype(np.float32)
    err = np.abs(kf - r)
    # dequant uses the fp16 scale: allow the fp16 rounding of s times the code
    assert (err <= 0.5 * s32[:, None] * (1 + 1e-3) + 15 * np.abs(s32 - s.astype(np.float32))[:, None] + 1e-6).all()
    codes = np.rint(r / np.where(s.astype(np.float32) == 0, 1, s.astype(np.float32))[:, None] + z.astype(np.float32)[:, None])
    amin = kf.argmin(1)
    assert (codes[np.arange(64), amin] == 0).all()


def test_c_matches_numpy_restatement():
    rng = np.random.default_rng(3)
    for trial in range(30):
        D, G = [(128, 128), (16, 8), (64, 32)][trial % 3]
        scale = [0.01, 1.0, 8.0, 300.0][trial % 4]
        k = (rng.standard_normal((D, G)) * scale).astype(np.float16)
        if trial % 5 == 0:
            k[3] = 1.25  # constant channel
        dk = max(1, D // 8)
        bi = _boost(D, dk, dk + 1, channels=rng.permutation(D)[:dk])
        a = O.quantize_key(k, bi, dk, dk + 1)
        b = O.quantize_key_np(k, bi, dk, dk + 1)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        assert np.array_equal(a[2].view(np.uint16), b[2].view(np.uint16))      # bits, sign of zero included
        assert np.array_equal(a[3].view(np.uint16), b[3].view(np.uint16))
        assert np.array_equal(O.dequantize_key(*a, bi, dk), O.dequantize_key_np(*a, bi, dk))
        va, vb = O.quantize_value(k.T.copy()), O.quantize_value_np(k.T.copy())
        for x, y in zip(va, vb):
            assert np.array_equal(np.asarray(x).view(np.uint8), np.asarray(y).view(np.uint8))
        assert np.array_equal(O.dequantize_value(*va), O.dequantize_value_np(*va))


def test_f2h_matches_numpy_rounding():
    rng = np.random.default_rng(4)
    xs = (rng.standard_normal(5000) * 10.0 ** rng.integers(-9, 5, 5000)).astype(np.float32)
    xs = np.concatenate([xs, np.float32([6.1035156e-05, 5.9604645e-08, 2.9802322e-08, 65504, 65519.99, 65520])])
    L = O.lib()
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.kitty_oracle_f2h(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, ref)


def make_paged_case(rng, H, Hq, D, G, d_boost, n_pages, n_sink, n_tail, P=None, outlier=8.0):
    """Quantise random K/V pages with the oracle into layout-shaped pools."""
    P = P or n_pages + 3
    sentinel = min(d_boost + 1, 255)
    kb = np.zeros((P, H, D, G // 4), np.uint8)
    kh = np.zeros((P, H, d_boost, G // 4), np.uint8)
    km = np.zeros((P, H, 2, D), np.float16)
    vp = np.zeros((P, H, G, D // 4), np.uint8)
    vm = np.zeros((P, H, G, 2), np.float16)
    bi = np.stack([_boost(D, d_boost, sentinel, channels=rng.permutation(D)[:d_boost]) for _ in range(H)])
    pages = rng.permutation(P)[:n_pages].astype(np.int32)
    for p in pages:
        for h in range(H):
            k = rng.standard_normal((D, G)).astype(np.float32)
            k[bi[h] < sentinel] *= outlier
            t2b, th, s, z = O.quantize_key(k.astype(np.float16), bi[h], d_boost, sentinel)
            kb[p, h], kh[p, h], km[p, h, 0], km[p, h, 1] = t2b, th, s, z
            pk, sv, zv = O.quantize_value(rng.standard_normal((G, D)).astype(np.float16))
            vp[p, h], vm[p, h, :, 0], vm[p, h, :, 1] = pk, sv, zv
    q = rng.standard_normal((Hq, D)).astype(np.float16)
    sk = rng.standard_normal((H, n_sink, D)).astype(np.float16)
    sv_ = rng.standard_normal((H, n_sink, D)).astype(np.float16)
    tk = rng.standard_normal((H, n_tail, D)).astype(np.float16)
    tv = rng.standard_normal((H, n_tail, D)).astype(np.float16)
    return dict(q=q, pages=pages, kb=kb, kh=kh, km=km, vp=vp, vm=vm, bi=bi, d_boost=d_boost,
                sk=sk, sv=sv_, tk=tk, tv=tv)


@pytest.mark.parametrize("H,Hq,n_pages,n_sink,n_tail", [(2, 2, 3, 4, 5), (2, 8, 2, 0, 3), (1, 4, 0, 3, 0),
                                                         (2, 4, 4, 2, 0)])
def test_paged_attention_matches_sdpa(H, Hq, n_pages, n_sink, n_tail):
    rng = np.random.default_rng(5)
    D, G, dk = 16, 8, 4
    c = make_paged_case(rng, H, Hq, D, G, dk, n_pages, n_sink, n_tail)
    out = O.paged_attention(c["q"], c["pages"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"], c["bi"], dk,
                            c["sk"], c["sv"], c["tk"], c["tv"], Hq, H, D)
    Ks, Vs = O.dequantized_kv(c["pages"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"], c["bi"], dk,
                              c["sk"], c["sv"], c["tk"], c["tv"])
    g = Hq // H
    for qh in range(Hq):
        K = torch.from_numpy(Ks[qh // g]).double()
        V = torch.from_numpy(Vs[qh // g]).double()
        qv = torch.from_numpy(c["q"][qh].astype(np.float64))[None, None, None]
        ref = torch.nn.functional.scaled_dot_product_attention(qv, K[None, None], V[None, None])[0, 0, 0]
        assert np.allclose(out[qh].astype(np.float64), ref.numpy(), atol=2e-3, rtol=1e-2)


def test_paged_attention_empty_context_is_zero():
    rng = np.random.default_rng(6)
    c = make_paged_case(rng, 2, 4, 16, 8, 4, 0, 0, 0)
    out = O.paged_attention(c["q"], [], c["kb"], c["kh"], c["km"], c["vp"], c["vm"], c["bi"], 4,
                            c["sk"], c["sv"], c["tk"], c["tv"], 4, 2, 16)
    assert (out.astype(np.float32) == 0).all()


def test_zero_point_sign_follows_torch_minimum_maximum():
    """Where -min/scale rounds to -0.0 (all-positive channels / tokens) the
    reference stores whatever sign torch.maximum / torch.minimum give
    (quantize_key.py:86-87, quantize_value.py:69-73).  For zero-point vectors
    whose length is a multiple of the CPU vector width (every production
    shape: D, G multiples of 16) torch's vector path returns +0.0; the oracle
    must store exactly those bits.  torch's own routines decide here."""
    rng = np.random.default_rng(11)
    k = (rng.uniform(0.05, 2.0, (32, 16))).astype(np.float16)   # every value > 0
    k[:, 0] = 0.01                                              # small min -> -min/s in (-0.5, 0)
    bi = _boost(32, 4, 5)
    kt = torch.from_numpy(k).float()
    mq = torch.where(torch.from_numpy(bi) < 5, 15.0, 3.0)
    sc = (kt.max(1).values - kt.min(1).values).clamp(min=1e-8) / mq
    zr = (-kt.min(1).values / sc).round()
    assert torch.signbit(zr).all()                              # every zero point starts as -0.0
    zt = torch.minimum(torch.maximum(zr, torch.zeros_like(zr)), mq).half()
    for _, _, s_, z_ in (O.quantize_key(k, bi, 4, 5), O.quantize_key_np(k, bi, 4, 5)):
        assert np.array_equal(z_.view(np.uint16), zt.numpy().view(np.uint16))
        assert np.array_equal(s_.view(np.uint16), sc.half().numpy().view(np.uint16))
    v = k.T.copy()                                              # 16 tokens x 32 channels
    vt = torch.from_numpy(v).float()
    svt = (vt.max(1).values - vt.min(1).values).clamp(min=1e-8) / 3.0
    zr = (-vt.min(1).values / svt).round()
    assert torch.signbit(zr).any()
    zvt = torch.minimum(torch.maximum(zr, torch.zeros_like(zr)), torch.full_like(zr, 3.0)).half()
    for _, _, z_ in (O.quantize_value(v), O.quantize_value_np(v)):
        assert np.array_equal(np.asarray(z_).view(np.uint16), zvt.numpy().view(np.uint16))


def test_torch_restatement_matches_c_oracle():
    """oracle/torch_reference.py (the timed CPU baseline) against the C
    oracle: dequantised pages bit for bit (same fp32 operations), the decode
    output to within the fp32 summation order (a few fp16 ulp)."""
    import torch_reference as TR
    rng = np.random.default_rng(21)
    H, Hq, D, G, dk = 2, 8, 32, 16, 6
    c = make_paged_case(rng, H, Hq, D, G, dk, 3, 4, 5)
    t = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in c.items() if isinstance(v, np.ndarray)}
    for p in c["pages"]:
        for h in range(H):
            ref_k = O.dequantize_key(c["kb"][p, h], c["kh"][p, h], c["km"][p, h, 0], c["km"][p, h, 1], c["bi"][h], dk)
            got_k = TR.dequantize_key_page(t["kb"][p, h], t["kh"][p, h], t["km"][p, h, 0], t["km"][p, h, 1],
                                           t["bi"][h], dk).numpy()
            assert np.array_equal(got_k.view(np.uint32), np.asarray(ref_k, np.float32).view(np.uint32))
            ref_v = O.dequantize_value(c["vp"][p, h], c["vm"][p, h, :, 0], c["vm"][p, h, :, 1])
            got_v = TR.dequantize_value_page(t["vp"][p, h], t["vm"][p, h, :, 0], t["vm"][p, h, :, 1]).numpy()
            assert np.array_equal(got_v.view(np.uint32), np.asarray(ref_v, np.float32).view(np.uint32))
    ref = O.paged_attention(c["q"], c["pages"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"], c["bi"], dk,
                            c["sk"], c["sv"], c["tk"], c["tv"], Hq, H, D)
    got = TR.paged_attention(t["q"], [int(p) for p in c["pages"]], t["kb"], t["kh"], t["km"], t["vp"], t["vm"],
                             t["bi"], dk, t["sk"], t["sv"], t["tk"], t["tv"], Hq, H, D).numpy()
    assert np.allclose(got.astype(np.float32), ref.astype(np.float32), atol=2e-3, rtol=2e-3)
    empty = TR.paged_attention(t["q"], [], t["kb"], t["kh"], t["km"], t["vp"], t["vm"], t["bi"], dk,
                               t["sk"][:, :0], t["sv"][:, :0], t["tk"][:, :0], t["tv"][:, :0], Hq, H, D)
    assert (empty.float() == 0).all()


def test_torch_quantizers_match_c_oracle():
    """The torch restatements of quantize_key_page_torch /
    quantize_value_page_torch (timed as config 2's CPU baseline) give the C
    oracle's codes, scales and zero points bit for bit: outlier and plain
    channels, a constant key channel and value token, an all-zero token,
    boost ranks with a gap and one at the last rank."""
    import torch_reference as TR
    rng = np.random.default_rng(33)
    D, G, dk = 128, 128, 16
    for trial in range(4):
        key = (rng.standard_normal((D, G)) * rng.choice([1.0, 8.0], size=(D, 1))).astype(np.float16)
        key[5] = np.float16(0.75)                           # a constant channel
        bi = np.full(D, dk + 1, np.uint8)
        ranks = rng.permutation(dk)[:dk - trial]             # a gap in the ranks for trial > 0
        bi[rng.permutation(D)[:len(ranks)]] = ranks
        val = rng.standard_normal((G, D)).astype(np.float16)
        val[3] = np.float16(-1.5)                            # a constant token
        val[9] = 0                                           # an all-zero token
        want_k = O.quantize_key(key, bi, dk, dk + 1)
        got_k = TR.quantize_key_page(torch.from_numpy(key), torch.from_numpy(bi), dk, dk + 1)
        for w, g in zip(want_k, got_k):
            assert np.array_equal(np.asarray(w).view(np.uint8), g.numpy().view(np.uint8)), trial
        want_v = O.quantize_value(val)
        got_v = TR.quantize_value_page(torch.from_numpy(val))
        for w, g in zip(want_v, got_v):
            assert np.array_equal(np.asarray(w).view(np.uint8), g.numpy().view(np.uint8)), trial


@pytest.mark.parametrize("npk,npv,nk", [(4, 4, 5), (4, 2, 5), (3, 0, 0), (5, 3, 7)])
def test_split_stream_oracle(npk, npv, nk):
    """Independent key / value streams (a value local window): the first npv
    of npk pages carry values; the value rows of the other pages, followed
    by the nk key-tail tokens' values, are FP16 in tail_v.

    * tail_v holding exactly the dequantised values of pages npv..npk-1
      (already fp16-exact: the page is quantised from them, then its
      dequantised fp32 rows are rounded to fp16) gives the C oracle's
      all-pages output up to that rounding;
    * npv == npk with equal tails is the C oracle's output itself;
    * SDPA on the assembled streams gives the same output."""
    rng = np.random.default_rng(31 + npk + npv)
    H, Hq, D, G, dk = 2, 8, 32, 16, 6
    c = make_paged_case(rng, H, Hq, D, G, dk, npk, 3, nk)
    keys, vals = list(c["pages"]), list(c["pages"][:npv])
    moved = np.zeros((H, (npk - npv) * G, D), np.float16)
    for j, p in enumerate(c["pages"][npv:]):
        for h in range(H):
            moved[h, j * G:(j + 1) * G] = O.dequantize_value(c["vp"][p, h], c["vm"][p, h, :, 0],
                                                             c["vm"][p, h, :, 1]).astype(np.float16)
    tv = np.concatenate([moved, c["tv"]], 1)
    args = (c["kb"], c["kh"], c["km"], c["vp"], c["vm"], c["bi"], dk, c["sk"], c["sv"])
    got = O.paged_attention_kv(c["q"], keys, vals, *args, c["tk"], tv, Hq, H, D).astype(np.float32)
    # every page's values from the pools: equal up to the fp16 rounding of the moved rows
    ref_all = O.paged_attention(c["q"], c["pages"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"], c["bi"], dk,
                                c["sk"], c["sv"], c["tk"], c["tv"], Hq, H, D).astype(np.float32)
    assert np.allclose(got, ref_all, atol=3e-3, rtol=1e-2)
    same = O.paged_attention_kv(c["q"], keys, keys, *args, c["tk"], c["tv"], Hq, H, D).astype(np.float32)
    assert np.allclose(same, ref_all, atol=1e-3, rtol=1e-3)
    Ks, Vs = O.split_stream_kv(keys, vals, *args, c["tk"], tv)
    assert Ks[0].shape[0] == 3 + npk * G + nk
    for qh in range(Hq):
        K = torch.from_numpy(Ks[qh // (Hq // H)]).double()
        V = torch.from_numpy(Vs[qh // (Hq // H)]).double()
        qv = torch.from_numpy(c["q"][qh].astype(np.float64))[None, None, None]
        ref = torch.nn.functional.scaled_dot_product_attention(qv, K[None, None], V[None, None])[0, 0, 0]
        assert np.allclose(got[qh], ref.numpy(), atol=2e-3, rtol=1e-2)
    with pytest.raises(ValueError):
        O.split_stream_kv(keys, vals, *args, c["tk"], c["tv"][:, :0] if npv < npk else c["tv"][:, :1])
