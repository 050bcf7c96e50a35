"""GPU parity of the fused split-K paged decode against the CPU oracle
(paged_attention_reference restated, kitty/kernels/attention.py:46-189).

Bar: |out - oracle| <= 2e-3 + 1e-2 * |oracle| elementwise.
"""
import numpy as np
import pytest
import torch

import oracle as O
from kvgen import random_pools, ragged_lengths
from test_oracle import make_paged_case

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _close(got, ref, what=""):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    err = np.abs(got - ref) - (ATOL + RTOL * np.abs(ref))
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert (err <= 0).all(), f"{what}: max excess {err.max():.3g} (max |diff| {np.abs(got - ref).max():.3g})"


def _to(dev, *arrs):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in arrs]


@pytest.mark.parametrize("H,Hq,D,G,dk,n_pages,n_sink,n_tail", [
    (2, 2, 16, 8, 4, 3, 4, 5),      # reference test config (tests/test_attention.py:24-36)
    (2, 8, 16, 8, 4, 2, 0, 3),
    (1, 4, 16, 8, 4, 0, 3, 0),      # sinks only (test_attention.py:190-215)
    (2, 4, 128, 128, 16, 5, 32, 96),
    (8, 8, 128, 128, 16, 7, 32, 96),  # config 1 shape: ctx 1024 = 32 + 7*128 + 96 (MHA on the group-4 MFMA kernel)
    (4, 8, 128, 128, 16, 9, 32, 50),  # groups of 2 on the group-4 MFMA kernel
    (3, 3, 128, 128, 32, 20, 0, 128), # MHA, 25 % INT4, no sinks, a full tail
    (2, 6, 128, 128, 16, 6, 32, 40),  # groups of 3 -> 4
    (2, 12, 128, 128, 16, 5, 32, 7),  # groups of 6 -> 8
    (1, 12, 128, 128, 16, 4, 32, 60), # a group of 12 -> 16
    (2, 6, 64, 32, 8, 5, 3, 9),       # generic kernel, groups of 3 -> 4
    (1, 12, 16, 8, 4, 6, 4, 5),       # generic kernel, a group of 12 -> 16
    (1, 32, 128, 128, 16, 5, 32, 40), # multi-query attention: two sub-groups of 16
    (2, 40, 128, 128, 16, 4, 32, 9),  # groups of 20: sub-groups of 16 and 4
    (1, 24, 64, 32, 8, 5, 3, 9),      # generic kernel, a group of 24: 16 and 8
    (2, 16, 128, 128, 32, 3, 7, 0),
    (2, 8, 128, 128, 5, 4, 32, 60),   # boosted channels not a multiple of 8 (part of a K-high row pair unused)
    (2, 16, 128, 128, 24, 3, 32, 30), # 24 boosted channels at GQA 8
    (2, 4, 64, 32, 8, 6, 1, 31),
    (2, 4, 256, 128, 32, 2, 5, 17),   # generic kernel at the largest head_dim
    (1, 2, 128, 256, 16, 2, 3, 100),  # and the largest page
])
def test_paged_attention_single_sequence(dev, H, Hq, D, G, dk, n_pages, n_sink, n_tail):
    from kitty.kernels import paged_attention
    rng = np.random.default_rng(H * 100 + Hq + D)
    c = make_paged_case(rng, H, Hq, D, G, dk, n_pages, n_sink, n_tail)
    ref = O.paged_attention(c["q"], c["pages"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"], c["bi"], dk,
                            c["sk"], c["sv"], c["tk"], c["tv"], Hq, H, D)
    q, kb, kh, km, vp, vm, bi, sk, sv, tk, tv = _to(dev, c["q"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"],
                                                   c["bi"], c["sk"], c["sv"], c["tk"], c["tv"])
    out = paged_attention(q, [int(p) for p in c["pages"]], kb, kh, km, vp, vm, bi, dk, sk, sv, tk, tv, Hq, H, D)
    assert out.shape == (Hq, D) and out.dtype == torch.float16
    _close(out.cpu().numpy(), ref, "single")


def test_empty_context_gives_zeros(dev):
    from kitty.kernels import paged_attention
    rng = np.random.default_rng(0)
    c = make_paged_case(rng, 2, 4, 16, 8, 4, 0, 0, 0)
    q, kb, kh, km, vp, vm, bi, sk, sv, tk, tv = _to(dev, c["q"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"],
                                                   c["bi"], c["sk"], c["sv"], c["tk"], c["tv"])
    out = paged_attention(q, [], kb, kh, km, vp, vm, bi, 4, sk, sv, tk, tv, 4, 2, 16)
    assert (out.float() == 0).all()


def test_tail_length_mismatch_raises(dev):
    from kitty.kernels import paged_attention
    rng = np.random.default_rng(0)
    c = make_paged_case(rng, 2, 2, 16, 8, 4, 1, 4, 5)
    q, kb, kh, km, vp, vm, bi, sk, sv, tk, tv = _to(dev, c["q"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"],
                                                   c["bi"], c["sk"], c["sv"], c["tk"], c["tv"])
    with pytest.raises(RuntimeError, match="equal lengths"):
        paged_attention(q, [int(c["pages"][0])], kb, kh, km, vp, vm, bi, 4, sk, sv, tk, tv[:, :3], 2, 2, 16)


def _batched_case(dev, seed, B, Hq, H, D, G, dk, ctx, S=32, shuffle=True, pool_extra=7, bi_edit=None):
    """Random-encoding pools, ctx[b] tokens per sequence = S sinks + pages + tail.
    bi_edit(bi) may rewrite the boost ranks before the pools are drawn."""
    gen = torch.Generator().manual_seed(seed)
    sentinel = dk + 1
    bi = torch.full((H, D), sentinel, dtype=torch.uint8)
    for h in range(H):
        bi[h, torch.randperm(D, generator=gen)[:dk]] = torch.arange(dk, dtype=torch.uint8)
    if bi_edit is not None:
        bi_edit(bi)
    n_pages = [(c - S) // G for c in ctx]
    tails = [(c - S) % G for c in ctx]
    P = sum(n_pages) + pool_extra
    pools = random_pools(gen, P, H, D, G, dk, bi)
    perm = torch.randperm(P, generator=gen) if shuffle else torch.arange(P)
    W = max(max(n_pages), 1)
    bt = torch.zeros(B, W, dtype=torch.int32)
    off = 0
    for b in range(B):
        bt[b, :n_pages[b]] = perm[off:off + n_pages[b]].to(torch.int32)
        off += n_pages[b]
    T = max(max(tails), 1)
    q = torch.randn(B, Hq, D, generator=gen).half()
    sk = torch.randn(B, H, S, D, generator=gen).half()
    sv = torch.randn(B, H, S, D, generator=gen).half()
    tk = torch.randn(B, H, T, D, generator=gen).half()
    tv = torch.randn(B, H, T, D, generator=gen).half()
    cpu = dict(q=q, bt=bt, n_pages=n_pages, tails=tails, pools=pools, bi=bi, sk=sk, sv=sv, tk=tk, tv=tv, S=S)
    return cpu


def _run_batched(dev, c, pages_per_split=0):
    from kitty.kernels import paged_attention_batched
    kb, kh, km, vp, vm = [t.to(dev) for t in c["pools"]]
    B = c["q"].shape[0]
    out = paged_attention_batched(
        c["q"].to(dev), c["bt"].to(dev), torch.tensor(c["n_pages"], dtype=torch.int32, device=dev),
        kb, kh, km, vp, vm, c["bi"].to(dev), c["sk"].to(dev), c["sv"].to(dev),
        torch.full((B,), c["S"], dtype=torch.int32, device=dev), c["tk"].to(dev), c["tv"].to(dev),
        torch.tensor(c["tails"], dtype=torch.int32, device=dev), pages_per_split=pages_per_split)
    return out.cpu().numpy()


def _oracle_batched(c, Hq, H, D, b):
    kb, kh, km, vp, vm = [t.numpy() for t in c["pools"]]
    n, t = c["n_pages"][b], c["tails"][b]
    return O.paged_attention(c["q"][b].numpy(), c["bt"][b, :n].numpy(), kb, kh, km, vp, vm, c["bi"].numpy(),
                             kh.shape[2], c["sk"][b].numpy(), c["sv"][b].numpy(), c["tk"][b, :, :t].numpy(),
                             c["tv"][b, :, :t].numpy(), Hq, H, D)


@pytest.mark.parametrize("pps", [0, 1, 3, 64])
def test_batched_ragged_split_invariance(dev, pps):
    """Config-4-like ragged batch (scaled down), shuffled pages; the result must
    not depend on the split size."""
    B, Hq, H, D, G, dk = 6, 32, 8, 128, 128, 32
    ctx = [int(x) for x in ragged_lengths(4, B, 40, 3000)]
    ctx[0] = 32   # sinks only
    c = _batched_case(dev, 40, B, Hq, H, D, G, dk, ctx)
    out = _run_batched(dev, c, pps)
    for b in range(B):
        _close(out[b], _oracle_batched(c, Hq, H, D, b), f"b={b} pps={pps}")


@pytest.mark.parametrize("Hq,pps,pages", [(8, 16, 300), (8, 6, 300), (8, 3, 300), (8, 2, 300), (16, 3, 300),
                                          (8, 20, 300), (8, 10, 300), (8, 8, 300), (8, 4, 300), (8, 4, 340),
                                          (16, 5, 300)])
def test_merge_partial_counts(dev, Hq, pps, pages):
    """One long sequence cut into many partials per (sequence, KV head): at
    least pps units per wave over 300 pages and 6 FP16 units gives 16, 20, 32,
    39, 52, 62, 78, 103 and 154 partials per pair for pps 20, 16, 10, 8, 6, 5,
    4, 3 and 2, and 340 pages at pps 4 give 88.  That takes the merge through
    every unrolled instance of its four-partials-per-load path (up to 16, 24,
    32, 48, 64, 80 and 96 partials, with 16 and 32 exactly at a bound), its
    float2 path for 128 and its two-pass path, for GQA groups of 4 and 8."""
    B, H, D, G, dk = 1, 2, 128, 128, 16
    c = _batched_case(dev, 50 + pps + pages, B, Hq, H, D, G, dk, [32 + pages * 128 + 50])
    out = _run_batched(dev, c, pps)
    _close(out[0], _oracle_batched(c, Hq, H, D, 0), f"Hq={Hq} pps={pps} pages={pages}")


@pytest.mark.parametrize("case", ["gqa16", "b70_uniform", "b70_ragged", "no_boost", "page_count_poison"])
def test_mfma_plan_edge_cases(dev, case):
    """Shapes the MFMA kernel's work plan treats specially, against the
    oracle: GQA 16 (one wave per SIMD, its own q set-up), more than 64
    sequences (the plan scans the batch 64 sequences at a time; uniform and
    ragged), no boosted channels, and a page count above max_pages (that
    sequence's output is NaN, the others are unaffected)."""
    D, G = 128, 128
    if case == "gqa16":
        B, Hq, H, dk = 3, 32, 2, 16
        ctx = [32 + 5 * 128 + 10, 32 + 40 * 128 + 100, 32]
    elif case == "b70_uniform":
        B, Hq, H, dk = 70, 8, 2, 16
        ctx = [32 + 3 * 128 + 20] * B
    elif case == "b70_ragged":
        B, Hq, H, dk = 70, 8, 2, 16
        ctx = [int(x) for x in ragged_lengths(7, B, 32, 32 + 12 * 128)]
    elif case == "no_boost":
        B, Hq, H, dk = 2, 16, 2, 0
        ctx = [32 + 9 * 128 + 7, 32 + 2 * 128 + 127]
    else:
        B, Hq, H, dk = 3, 8, 2, 16
        ctx = [32 + 4 * 128 + 3, 32 + 4 * 128 + 3, 32 + 2 * 128]
    c = _batched_case(dev, 60 + len(case), B, Hq, H, D, G, dk, ctx)
    if case == "page_count_poison":
        c["n_pages"][1] = c["bt"].shape[1] + 1   # above max_pages (the table width)
    out = _run_batched(dev, c)
    for b in range(B):
        if case == "page_count_poison" and b == 1:
            assert np.isnan(out[b]).all()
            continue
        _close(out[b], _oracle_batched(c, Hq, H, D, b), f"{case} b={b}")


@pytest.mark.parametrize("name,B,Hq,H,ctx,dk", [
    ("config3", 16, 32, 8, 32768, 16),
    ("config5", 4, 64, 8, 131072, 16),
])
def test_full_size_configs(dev, name, B, Hq, H, ctx, dk):
    """BASELINE configs 3 and 5 at their full shapes against the oracle
    (every sequence, every head)."""
    D, G = 128, 128
    c = _batched_case(dev, 3 if name == "config3" else 5, B, Hq, H, D, G, dk, [ctx] * B, pool_extra=11)
    out = _run_batched(dev, c)
    for b in range(B):
        _close(out[b], _oracle_batched(c, Hq, H, D, b), f"{name} b={b}")


def test_repeated_launches_are_bit_identical(dev):
    """The split kernel, the merge and the plan use no atomics and no
    run-time work claiming, so a decode gives the same bits on every launch,
    also when other decodes (another plan and shape, GQA 8) run in between.
    Checked for the GQA-4 and GQA-8 kernels on ragged batches."""
    cases = [_batched_case(dev, 91, 5, 32, 8, 128, 128, 16, [32 + 37 * 128 + 5, 32 + 11 * 128 + 90, 32 + 60 * 128,
                                                            32 + 2 * 128 + 17, 32 + 25 * 128 + 127]),
             _batched_case(dev, 92, 3, 16, 2, 128, 128, 32, [32 + 50 * 128 + 64, 32 + 9 * 128 + 3, 32 + 70 * 128 + 1])]
    first = [_run_batched(dev, c) for c in cases]
    for _ in range(3):
        for c, ref in zip(cases, first):
            out = _run_batched(dev, c)
            assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


def _random_shape(rnd):
    """One seeded decode shape: the MFMA kernel (D = G = 128, any boosted
    channel count up to 32) or the generic one, any GQA group up to 32, up
    to 160 pages, batches past 64 sequences, sink counts 0-32, split sizes."""
    if rnd.random() < 0.7:
        D = G = 128
        dk = rnd.choice([0, 1, 5, 8, 16, 17, 24, 31, 32])
        maxp = rnd.choice([1, 3, 8, 20, 40, 90, 160])
    else:
        D, G = rnd.choice([16, 32, 64, 128, 256]), rnd.choice([8, 16, 32, 64, 128, 256])
        dk = rnd.choice([0, 1, min(4, D), min(D // 8, 32), min(D // 4, 32)])
        maxp = rnd.choice([1, 2, 5, 9])
    H = rnd.choice([1, 2, 4, 8])
    Hq = H * rnd.choice([1, 2, 3, 4, 5, 6, 8, 12, 16, 20, 24, 32])
    B = rnd.choice([1, 2, 3, 5, 9, 17]) if rnd.random() < 0.9 else rnd.choice([65, 70])
    if B > 20:
        maxp = min(maxp, 3)
    if maxp > 40:
        B = min(B, 3)
    S = rnd.choice([0, 1, 7, 32])
    ctx = [S + rnd.randint(0, maxp * G + G - 1) for _ in range(B)]
    return D, G, dk, H, Hq, B, S, ctx, rnd.choice([0, 0, 0, 1, 3, 7, 64])


def test_random_shapes_match_oracle(dev):
    """120 seeded random shapes through the batched decode against the
    oracle (up to six sequences of each checked)."""
    import random
    for k in range(120):
        rnd = random.Random(7000 + k)
        D, G, dk, H, Hq, B, S, ctx, pps = _random_shape(rnd)
        what = f"seed {7000 + k}: D{D} G{G} dk{dk} H{H} Hq{Hq} B{B} S{S} pages_per_split {pps}"
        c = _batched_case(dev, 7000 + k, B, Hq, H, D, G, dk, ctx, S=S)
        out = _run_batched(dev, c, pages_per_split=pps)
        for b in (range(B) if B <= 6 else rnd.sample(range(B), 6)):
            _close(out[b], _oracle_batched(c, Hq, H, D, b), what + f" b={b}")


def test_duplicate_boost_ranks_take_the_generic_path(dev):
    """Channels sharing a boost rank read the same high-bit row back
    (dequantize_key.py:70-87) and a channel ranked D_boost has none: the MFMA
    kernel assumes one channel per rank, so the batched decode detects the
    repeated rank and runs the generic kernel, which matches the oracle."""
    from kitty.kernels.ops import boost_rows_unique

    def edit(bi):
        r0, r1 = (bi[0] == 0).nonzero()[0, 0], (bi[0] == 1).nonzero()[0, 0]
        assert r0 != r1
        bi[0, r1] = 0                                    # rank 0 twice in head 0
        bi[3, (bi[3] == 17).nonzero()[0, 0]] = 16        # head 3: one channel ranked D_boost
    c = _batched_case(dev, 41, 3, 32, 8, 128, 128, 16, [32 + 128 * 5 + 17, 32 + 128 * 3, 32 + 128 * 9 + 100],
                      bi_edit=edit)
    assert not boost_rows_unique(c["bi"], 16)
    out = _run_batched(dev, c)
    for b in range(3):
        _close(out[b], _oracle_batched(c, 32, 8, 128, b), f"dup b={b}")


def test_invalid_page_id_poisons_output(dev):
    """A page id outside the pool is never dereferenced; the sequence's output becomes NaN."""
    B, Hq, H, D, G, dk = 2, 4, 2, 128, 128, 16
    c = _batched_case(dev, 9, B, Hq, H, D, G, dk, [32 + 3 * 128 + 5, 32 + 2 * 128])
    c["bt"][1, 1] = 10 ** 6
    out = _run_batched(dev, c)
    assert np.isnan(out[1]).all()
    _close(out[0], _oracle_batched(c, Hq, H, D, 0), "b=0")


def test_large_query_times_key_scale_stays_finite(dev):
    """|q[d] s_k[d]| past the fp16 maximum (65,504) but below the documented
    2^17 / 2^19 bounds: the MFMA kernel's 2^-3 prescaled QK operand stays
    finite and the output matches the oracle's fp32 scores (here up to
    |q s| ~ 1.8e5 on the INT2 channels, 3.6e4 on the INT4 ones; the softmax
    picks one token)."""
    from kitty.kernels import paged_attention
    rng = np.random.default_rng(77)
    H, Hq, D, G, dk, n_pages = 2, 8, 128, 128, 16, 4
    sentinel = dk + 1
    c = make_paged_case(rng, H, Hq, D, G, dk, n_pages, 32, 20)
    for p in c["pages"]:
        for h in range(H):
            k = (rng.standard_normal((D, G)) * 600.0).astype(np.float16)
            c["kb"][p, h], c["kh"][p, h], c["km"][p, h, 0], c["km"][p, h, 1] = O.quantize_key(k, c["bi"][h], dk,
                                                                                               sentinel)
    c["q"] = (rng.standard_normal((Hq, D)) * 40.0).astype(np.float16)
    qs = np.abs(c["q"].astype(np.float64)).max() * np.abs(c["km"][c["pages"], :, 0].astype(np.float64)).max()
    assert 65504 < qs < 2 ** 19
    ref = O.paged_attention(c["q"], c["pages"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"], c["bi"], dk,
                            c["sk"], c["sv"], c["tk"], c["tv"], Hq, H, D)
    assert np.isfinite(ref.astype(np.float32)).all()
    q, kb, kh, km, vp, vm, bi, sk, sv, tk, tv = _to(dev, c["q"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"],
                                                   c["bi"], c["sk"], c["sv"], c["tk"], c["tv"])
    out = paged_attention(q, [int(p) for p in c["pages"]], kb, kh, km, vp, vm, bi, dk, sk, sv, tk, tv, Hq, H, D)
    _close(out.cpu().numpy(), ref, "large q s_k")


def test_config4_ragged_batch_64bit_offsets(dev):
    """BASELINE config 4 at full size: 64 sequences with seeded ragged
    contexts in [512, 65536], 32 query / 8 KV heads, 25% INT4 channels
    (D_boost = 32), pages scattered by a shuffled free list over a
    70,000-page pool, so page ids beyond 65,536 put key / value byte offsets
    past 2^31 (64-bit addressing).  Every sequence and head against the oracle."""
    from kitty.kernels import paged_attention_batched
    B, Hq, H, D, G, dk, S = 64, 32, 8, 128, 128, 32, 32
    P_dev = 70_000
    ctx = [int(x) for x in ragged_lengths(4, B, 512, 65536)]
    n_pages = [(c - S) // G for c in ctx]
    tails = [(c - S) % G for c in ctx]
    U = sum(n_pages)
    gen = torch.Generator().manual_seed(44)
    bi = torch.full((H, D), dk + 1, dtype=torch.uint8)
    for h in range(H):
        bi[h, torch.randperm(D, generator=gen)[:dk]] = torch.arange(dk, dtype=torch.uint8)
    host = random_pools(gen, U, H, D, G, dk, bi, rng=np.random.default_rng(44))  # compact: list page u = row u
    ids = torch.randperm(P_dev, generator=gen)[:U]               # shuffled free list
    assert int(ids.max()) >= 65_536                              # some byte offsets exceed 2^31
    shapes = [(P_dev,) + tuple(t.shape[1:]) for t in host]
    pools = [torch.empty(s, dtype=t.dtype, device=dev) for s, t in zip(shapes, host)]
    ids_dev = ids.to(dev)
    for pd, t in zip(pools, host):
        pd.index_copy_(0, ids_dev, t.to(dev))
    W = max(n_pages)
    bt = torch.zeros(B, W, dtype=torch.int32)
    bt_compact = torch.zeros(B, W, dtype=torch.int32)
    off = 0
    for b in range(B):
        bt[b, :n_pages[b]] = ids[off:off + n_pages[b]].to(torch.int32)
        bt_compact[b, :n_pages[b]] = torch.arange(off, off + n_pages[b], dtype=torch.int32)
        off += n_pages[b]
    T = max(tails)
    q = torch.randn(B, Hq, D, generator=gen).half()
    sk, sv = torch.randn(B, H, S, D, generator=gen).half(), torch.randn(B, H, S, D, generator=gen).half()
    tk, tv = torch.randn(B, H, T, D, generator=gen).half(), torch.randn(B, H, T, D, generator=gen).half()
    out = paged_attention_batched(
        q.to(dev), bt.to(dev), torch.tensor(n_pages, dtype=torch.int32, device=dev), *pools, bi.to(dev),
        sk.to(dev), sv.to(dev), torch.full((B,), S, dtype=torch.int32, device=dev), tk.to(dev), tv.to(dev),
        torch.tensor(tails, dtype=torch.int32, device=dev)).cpu().numpy()
    del pools
    kb, kh, km, vp, vm = [t.numpy() for t in host]
    for b in range(B):
        n, t = n_pages[b], tails[b]
        ref = O.paged_attention(q[b].numpy(), bt_compact[b, :n].numpy(), kb, kh, km, vp, vm, bi.numpy(), dk,
                                sk[b].numpy(), sv[b].numpy(), tk[b, :, :t].numpy(), tv[b, :, :t].numpy(), Hq, H, D)
        _close(out[b], ref, f"config4 b={b} ctx={ctx[b]}")


@pytest.mark.parametrize("kernel,Hq,H,D,G,dk", [("mfma", 32, 8, 128, 128, 16), ("mfma", 64, 8, 128, 128, 32),
                                               ("mfma", 128, 8, 128, 128, 16), ("generic", 8, 4, 64, 32, 8)])
def test_independent_value_stream(dev, kernel, Hq, H, D, G, dk):
    """Key and value streams of different page counts (P_v <= P_k, the value
    local window of the pipeline): the value rows of key pages P_v..P_k-1 and
    of the key tail come from tail_v, (P_k - P_v) G + tail_len rows of it.
    Against the oracle's split-stream decode, per sequence and head, with
    P_v = P_k (the reference layout), P_v = P_k - 1 (a 128-token window),
    P_v = 0 (every value FP16) and P_v = P_k - 2; the MFMA kernel (key-only
    pages in its FP16 segments) at GQA 4, 8 and 16, and the generic kernel."""
    from kitty.kernels import paged_attention_batched
    S = 32 if D == 128 else 40
    ctx = [S + 6 * G + 17, S + 3 * G, S + 2 * G + G - 1, S + 1 * G + 5, S + 9 * G + 60]
    B = len(ctx)
    c = _batched_case(dev, 90 + Hq, B, Hq, H, D, G, dk, ctx, S=S)
    npk = c["n_pages"]
    npv = [npk[0], npk[1] - 1, 0, npk[3] - 1, npk[4] - 2]
    nv = [(a - b) * G + t for a, b, t in zip(npk, npv, c["tails"])]
    gen = torch.Generator().manual_seed(7)
    tv = torch.randn(B, H, max(nv), D, generator=gen).half()
    kb, kh, km, vp, vm = [t.to(dev) for t in c["pools"]]
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    print(f"value stream {kernel} Hq={Hq}: npk={npk} npv={npv} nv={nv}", flush=True)
    out = paged_attention_batched(
        c["q"].to(dev), c["bt"].to(dev), i32(npk), kb, kh, km, vp, vm, c["bi"].to(dev), c["sk"].to(dev),
        c["sv"].to(dev), i32([S] * B), c["tk"].to(dev), tv.to(dev), i32(c["tails"]),
        num_pages_v=i32(npv), tail_len_v=i32(nv)).cpu().numpy()
    pools = [t.numpy() for t in c["pools"]]
    for b in range(B):
        bt = c["bt"][b].numpy()
        ref = O.paged_attention_kv(c["q"][b].numpy(), bt[:npk[b]], bt[:npv[b]], *pools, c["bi"].numpy(), dk,
                                   c["sk"][b].numpy(), c["sv"][b].numpy(), c["tk"][b, :, :c["tails"][b]].numpy(),
                                   tv[b, :, :nv[b]].numpy(), Hq, H, D)
        _close(out[b], ref, f"{kernel} b={b} npk={npk[b]} npv={npv[b]}")


def test_value_stream_length_mismatch_poisons_sequence(dev):
    """A sequence whose value stream is not as long as its key stream
    ((P_k - P_v) G + tail_len != tail_len_v) gets NaN output; the others
    are unaffected."""
    from kitty.kernels import paged_attention_batched
    B, Hq, H, D, G, dk = 2, 32, 8, 128, 128, 16
    c = _batched_case(dev, 95, B, Hq, H, D, G, dk, [32 + 4 * 128 + 9, 32 + 3 * 128 + 2])
    npk, tails = c["n_pages"], c["tails"]
    npv = [npk[0] - 1, npk[1] - 1]
    nv = [128 + tails[0], 128 + tails[1] - 1]            # sequence 1 one row short
    tv = torch.randn(B, H, max(nv), D, generator=torch.Generator().manual_seed(3)).half()
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    kb, kh, km, vp, vm = [t.to(dev) for t in c["pools"]]
    out = paged_attention_batched(
        c["q"].to(dev), c["bt"].to(dev), i32(npk), kb, kh, km, vp, vm, c["bi"].to(dev), c["sk"].to(dev),
        c["sv"].to(dev), i32([32] * B), c["tk"].to(dev), tv.to(dev), i32(tails),
        num_pages_v=i32(npv), tail_len_v=i32(nv)).cpu().numpy()
    assert np.isnan(out[1]).all()
    bt = c["bt"][0].numpy()
    ref = O.paged_attention_kv(c["q"][0].numpy(), bt[:npk[0]], bt[:npv[0]], *[t.numpy() for t in c["pools"]],
                               c["bi"].numpy(), dk, c["sk"][0].numpy(), c["sv"][0].numpy(),
                               c["tk"][0, :, :tails[0]].numpy(), tv[0, :, :nv[0]].numpy(), Hq, H, D)
    _close(out[0], ref, "b=0")
