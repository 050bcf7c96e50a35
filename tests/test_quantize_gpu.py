"""GPU parity of the batch quantize + pack kernel against the CPU oracle.

Bar: packed codes bit-exact, scales and zero points equal by value (the sign
of a zero zero-point is the only unpinned bit, see oracle/oracle.py).
"""
import numpy as np
import pytest
import torch

import oracle as O
from kvgen import calibrate_boost_idx, outlier_keys

pytestmark = pytest.mark.gpu


def _eq16(a, b):
    """fp16 bit patterns equal (the sign of a zero zero-point included)."""
    return np.array_equal(np.ascontiguousarray(a, np.float16).view(np.uint16),
                          np.ascontiguousarray(b, np.float16).view(np.uint16))


def _pools(P, H, D, G, Dk, dev):
    from kitty.kernels.ops import pool_store
    kb = torch.full((P, H, D, G // 4), 0xAA, dtype=torch.uint8, device=dev)  # garbage: must be overwritten
    kh = torch.full((P, H, Dk, G // 4), 0x55, dtype=torch.uint8, device=dev)
    km = torch.full((P, H, 2, D), 7.0, dtype=torch.float16, device=dev)
    vp = torch.full((P, H, G, D // 4), 0x33, dtype=torch.uint8, device=dev)
    vm = torch.full((P, H, G, 2), 7.0, dtype=torch.float16, device=dev)
    return (kb, kh, km, vp, vm), pool_store(kb, kh, km, vp, vm)


def _check_page(pools, p, h, key_dg, value_gd, bi, Dk, sentinel, value_rows=None):
    kb, kh, km, vp, vm = [t.cpu().numpy() for t in pools]
    t2b, th, s, z = O.quantize_key(key_dg, bi, Dk, sentinel)
    assert np.array_equal(kb[p, h], t2b), (p, h)
    assert np.array_equal(kh[p, h], th), (p, h)
    assert _eq16(km[p, h, 0], s) and _eq16(km[p, h, 1], z), (p, h)
    if value_gd is not None:
        v = value_gd.copy()
        if value_rows is not None:
            v[value_rows:] = 0
        pk, sv, zv = O.quantize_value(v)
        assert np.array_equal(vp[p, h], pk), (p, h)
        assert _eq16(vm[p, h, :, 0], sv) and _eq16(vm[p, h, :, 1], zv), (p, h)


def test_config2_quantize_pack_bit_exact(dev):
    """4096 tokens x 8 KV heads x 128, 16 outlier key
    channels per head x8, per-channel keys over G=128 groups, per-token values,
    INT4 for the top 12.5% channels."""
    from kitty.kernels.ops import quantize_into_pools
    gen = torch.Generator().manual_seed(2)
    T, H, D, G, Dk = 4096, 8, 128, 128, 16
    sentinel = Dk + 1
    K, chans = outlier_keys(gen, (T,), H, D, 16, 8.0)
    V = torch.randn(T, H, D, generator=gen).half()
    calib, _ = outlier_keys(gen, (256,), H, D, 16, 8.0, channels=chans)
    bi = calibrate_boost_idx(calib, Dk, sentinel)
    n_groups = T // G
    P = n_groups + 5
    pools, store = _pools(P, H, D, G, Dk, dev)
    page_ids = torch.randperm(P, generator=gen)[:n_groups].to(torch.int32)
    Kd, Vd = K.to(dev), V.to(dev)
    kblocks = Kd.view(n_groups, G, H, D).permute(0, 2, 1, 3)   # (group, head, token, chan) strided
    vblocks = Vd.view(n_groups, G, H, D).permute(0, 2, 1, 3)
    quantize_into_pools(store, kblocks, vblocks, bi.to(dev), page_ids.to(dev), sentinel)
    torch.cuda.synchronize()
    Kn, Vn = K.numpy(), V.numpy()
    for g in range(n_groups):
        for h in range(H):
            _check_page(pools, int(page_ids[g]), h, Kn[g * G:(g + 1) * G, h].T.copy(),
                        Vn[g * G:(g + 1) * G, h].copy(), bi[h].numpy(), Dk, sentinel)


@pytest.mark.parametrize("D,G,Dk,H", [(16, 8, 4, 2), (128, 128, 32, 4), (64, 32, 15, 1), (32, 16, 0, 3),
                                     (256, 128, 32, 2), (128, 256, 16, 1)])   # D*G = 32768: > 64 KB of LDS
def test_small_shapes_and_edge_rows(dev, D, G, Dk, H):
    from kitty.kernels.ops import quantize_into_pools
    gen = torch.Generator().manual_seed(D * 7 + G)
    sentinel = min(Dk + 1, 255)
    n = 3
    K = torch.randn(n, H, G, D, generator=gen)
    K[0, 0, :, 1] = 2.5           # constant channel -> fp16 scale underflow
    K[1, 0] = 0.0                 # all-zero block
    K[2, -1, 0, :] = 0.5 * torch.arange(D)  # ties
    K[2, 0, :, 2] = 0.01 + torch.rand(G, generator=gen)   # positive channel: -min/s rounds to -0.0
    K = K.half()
    V = torch.randn(n, H, G, D, generator=gen).half()
    V[0, 0, 3] = -1.0             # constant token
    V[1, 0, 5] = (0.01 + torch.rand(D, generator=gen)).half()  # positive token: zero point -0.0 -> +0.0
    bi = torch.full((n, H, D), sentinel, dtype=torch.uint8)
    for o in range(n):
        for h in range(H):
            perm = torch.randperm(D, generator=gen)[:Dk]
            bi[o, h, perm] = torch.arange(Dk, dtype=torch.uint8)
    pools, store = _pools(n + 1, H, D, G, Dk, dev)
    page_ids = torch.tensor([2, 0, 3], dtype=torch.int32)
    quantize_into_pools(store, K.to(dev), V.to(dev), bi.to(dev), page_ids.to(dev), sentinel)
    torch.cuda.synchronize()
    for o in range(n):
        for h in range(H):
            _check_page(pools, int(page_ids[o]), h, K[o, h].numpy().T.copy(), V[o, h].numpy(), bi[o, h].numpy(),
                        Dk, sentinel)


def _random_blocks(rnd, gen, n, H, G, D):
    """(n, H, G, D) fp16 blocks from one of several seeded distributions:
    normal at a random power-of-two scale (fp16 subnormals to ~2^14), a
    half-integer grid (every element a tie of some scale), heavy tails,
    outlier channels, constant tokens / channels."""
    kind = rnd.choice(["normal", "grid", "heavy", "outlier", "flat"])
    x = torch.randn(n, H, G, D, generator=gen)
    if kind == "normal":
        x = x * 2.0 ** rnd.randint(-20, 12)
    elif kind == "grid":
        x = torch.round(x * 4) / 2 * 2.0 ** rnd.randint(-6, 6)
    elif kind == "heavy":
        x = x / torch.rand(n, H, G, D, generator=gen).clamp(min=1e-3).sqrt()
    elif kind == "outlier":
        x[..., torch.randperm(D, generator=gen)[: max(1, D // 8)]] *= 16.0
    else:
        x[:, :, rnd.randrange(G)] = 1.25
        x[..., rnd.randrange(D)] = -3.0
    return x.clamp(-60000, 60000).half()


def test_random_blocks_bit_exact(dev):
    """40 seeded random batches (shape, boosted channels, value rows and data
    distribution drawn per case) through the batch kernel: every page
    bit-exact against the oracle."""
    import random
    from kitty.kernels.ops import quantize_into_pools
    for k in range(40):
        rnd = random.Random(900 + k)
        gen = torch.Generator().manual_seed(900 + k)
        D, G = rnd.choice([(128, 128)] * 5 + [(16, 8), (64, 32), (32, 16), (256, 128), (128, 256)])
        Dk = rnd.choice([0, 1, 5, 16, 31, 32]) if D >= 32 else rnd.choice([0, 1, 4])
        H, n = rnd.choice([1, 2, 8]), rnd.choice([1, 3, 9])
        sentinel = min(Dk + 1, 255)
        rows = rnd.choice([None, None, 0, 1, G // 2, G - 1])
        K = _random_blocks(rnd, gen, n, H, G, D)
        V = _random_blocks(rnd, gen, n, H, G, D)
        bi = torch.full((n, H, D), sentinel, dtype=torch.uint8)
        for o in range(n):
            for h in range(H):
                bi[o, h, torch.randperm(D, generator=gen)[:Dk]] = torch.arange(Dk, dtype=torch.uint8)
        pools, store = _pools(n + 2, H, D, G, Dk, dev)
        page_ids = torch.randperm(n + 2, generator=gen)[:n].to(torch.int32)
        quantize_into_pools(store, K.to(dev), V.to(dev), bi.to(dev), page_ids.to(dev), sentinel, value_rows=rows)
        torch.cuda.synchronize()
        for o in range(n):
            for h in range(H):
                _check_page(pools, int(page_ids[o]), h, K[o, h].numpy().T.copy(), V[o, h].numpy(),
                            bi[o, h].numpy(), Dk, sentinel, value_rows=rows)


def test_duplicate_and_rowless_boost_ranks(dev):
    """Channels sharing a boost rank OR their high bits into the rank's row,
    and a channel ranked D_boost (below the sentinel) gets INT4 codes with no
    high row (quantize_key.py:73, 113-119); 128 x 128 kernel, bit-exact."""
    from kitty.kernels.ops import quantize_into_pools
    D = G = 128
    H, Dk, sentinel = 2, 16, 17
    gen = torch.Generator().manual_seed(77)
    K = torch.randn(1, H, G, D, generator=gen).half()
    bi = torch.full((1, H, D), sentinel, dtype=torch.uint8)
    for h in range(H):
        ch = torch.randperm(D, generator=gen)[:Dk + 1]
        bi[0, h, ch[:Dk]] = torch.arange(Dk, dtype=torch.uint8)
        bi[0, h, ch[1]] = 0      # rank 0 three times, ranks 1 and 2 unused (their rows stay 0)
        bi[0, h, ch[2]] = 0
        bi[0, h, ch[Dk]] = Dk    # INT4 codes, high bits not stored
    pools, store = _pools(1, H, D, G, Dk, dev)
    quantize_into_pools(store, K.to(dev), None, bi.to(dev), torch.zeros(1, dtype=torch.int32, device=dev),
                        sentinel)
    torch.cuda.synchronize()
    for h in range(H):
        _check_page(pools, 0, h, K[0, h].numpy().T.copy(), None, bi[0, h].numpy(), Dk, sentinel)


def _boundary_block(gen, G, D, mq_of_col):
    """fp16 values at and one fp16 ulp either side of the rounding boundaries
    (j + 1/2) * s of rint(x / s), for exact (s = 1) and inexact (s = 1/3,
    2/15, ...) scales; column c is a group with max code mq_of_col[c] whose
    min / max are pinned to -rng/2, +rng/2."""
    x = np.zeros((G, D), np.float16)
    for c in range(D):
        mq = mq_of_col[c]
        rng = [float(mq), 1.0, 2.0, 0.7][c % 4]
        s = np.float32(rng) / np.float32(mq)
        j = torch.randint(-(mq + 1) // 2, (mq - 1) // 2 + 1, (G,), generator=gen).numpy()
        t = ((j + 0.5) * s).astype(np.float16)
        step = torch.randint(-1, 2, (G,), generator=gen).numpy()
        col = np.where(step == 0, t, np.where(step > 0, np.nextafter(t, np.float16(np.inf)),
                                              np.nextafter(t, np.float16(-np.inf))))
        col[0], col[1] = -rng / 2, rng / 2
        x[:, c] = col
    return x


def test_rounding_boundaries_bit_exact(dev):
    """Values on and next to the half-integer code boundaries: the kernel's
    multiply-by-reciprocal codes must take the exact-division path there and
    match the correctly rounded quotient (quantize_key.py:95, quantize_value.py:79)."""
    from kitty.kernels.ops import quantize_into_pools
    D, G, H, Dk = 128, 128, 2, 32
    gen = torch.Generator().manual_seed(77)
    bi = torch.full((H, D), Dk + 1, dtype=torch.uint8)
    for h in range(H):
        bi[h, torch.randperm(D, generator=gen)[:Dk]] = torch.arange(Dk, dtype=torch.uint8)
    K = np.stack([_boundary_block(gen, G, D, [15 if bi[h, c] < Dk + 1 else 3 for c in range(D)])
                  for h in range(H)])                                     # (H, G, D) token-major
    V = np.stack([_boundary_block(gen, D, G, [3] * G).T.copy() for h in range(H)])  # per-token groups
    pools, store = _pools(2, H, D, G, Dk, dev)
    quantize_into_pools(store, torch.from_numpy(K)[None].to(dev), torch.from_numpy(V)[None].to(dev), bi.to(dev),
                        torch.tensor([1], dtype=torch.int32, device=dev), Dk + 1)
    torch.cuda.synchronize()
    for h in range(H):
        _check_page(pools, 1, h, K[h].T.copy(), V[h], bi[h].numpy(), Dk, Dk + 1)


@pytest.mark.parametrize("rows", [0, 1, 37, 127])
def test_value_rows_zero_padding(dev, rows):
    """Rows past value_rows quantise as zeros (pipeline.py:240-243); the
    128 x 128 kernel reads them from a zero row, not from the source."""
    from kitty.kernels.ops import quantize_into_pools
    D, G, H = 128, 128, 2
    gen = torch.Generator().manual_seed(11 + rows)
    V = torch.randn(1, H, G, D, generator=gen).half()
    pools, store = _pools(1, H, D, G, 16, dev)
    quantize_into_pools(store, None, V.to(dev), None, torch.zeros(1, dtype=torch.int32, device=dev), 17,
                        value_rows=rows)
    torch.cuda.synchronize()
    vp, vm = pools[3].cpu().numpy(), pools[4].cpu().numpy()
    for h in range(H):
        v = V[0, h].numpy().copy()
        v[rows:] = 0
        pk, sv, zv = O.quantize_value(v)
        assert np.array_equal(vp[0, h], pk) and _eq16(vm[0, h, :, 0], sv) and _eq16(vm[0, h, :, 1], zv)


@pytest.mark.parametrize("D,G,Dk,H,S,n", [(128, 128, 16, 8, 32, 3), (128, 128, 32, 2, 0, 2), (64, 32, 8, 3, 5, 4)])
def test_pages_read_in_place_from_a_prompt(dev, D, G, Dk, H, S, n):
    """(n_seq, pages, H, G, D) views of a (B, H, T, D) prompt, quantised in
    place with the sequence stride (outer_per_seq): every page bit-exact
    against the oracle on the same tokens, and pools identical to the launch
    over the same blocks copied out page-major (128 x 128 kernel for the first
    two shapes, the shape-generic kernel for the last)."""
    from kitty.kernels.ops import quantize_into_pools
    gen = torch.Generator().manual_seed(D + G + S + n)
    B, sentinel = 3, Dk + 1
    Tt = S + n * G + 7
    K, chans = outlier_keys(gen, (B, Tt), H, D, max(Dk, 1), 8.0)
    K = K.permute(0, 2, 1, 3).contiguous()                    # (B, H, T, D)
    V = torch.randn(B, H, Tt, D, generator=gen).half()
    bi = torch.full((H, D), sentinel, dtype=torch.uint8)
    for h in range(H):
        bi[h, torch.randperm(D, generator=gen)[:Dk]] = torch.arange(Dk, dtype=torch.uint8)
    P = B * n + 4
    page_ids = torch.randperm(P, generator=gen)[:B * n].to(torch.int32).to(dev)
    Kd, Vd, bid = K.to(dev), V.to(dev), bi.to(dev)
    view = lambda x: x[:, :, S:S + n * G].unflatten(2, (n, G)).transpose(1, 2)   # (B, n, H, G, D), no copy
    pools, store = _pools(P, H, D, G, Dk, dev)
    quantize_into_pools(store, view(Kd), view(Vd), bid, page_ids, sentinel)
    pools2, store2 = _pools(P, H, D, G, Dk, dev)
    flat = lambda x: view(x).reshape(B * n, H, G, D)          # the page-major copy
    quantize_into_pools(store2, flat(Kd), flat(Vd), bid, page_ids, sentinel)
    torch.cuda.synchronize()
    for a, b in zip(pools, pools2):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    Kn, Vn, ids = K.numpy(), V.numpy(), page_ids.cpu().numpy()
    for b in range(B):
        for p in range(n):
            t0 = S + p * G
            for h in range(H):
                _check_page(pools, int(ids[b * n + p]), h, Kn[b, h, t0:t0 + G].T.copy(), Vn[b, h, t0:t0 + G].copy(),
                            bi[h].numpy(), Dk, sentinel)


def test_reference_signatures(dev):
    """quantize_key_page / quantize_value_page / dequantize_* with the
    reference's arguments, outputs written into strided pool views."""
    from kitty.kernels import (quantize_key_page, quantize_value_page, quantize_key_page_torch,
                               quantize_value_page_torch, dequantize_key_page_torch, dequantize_value_page_torch,
                               dequantize_key_page)
    D, G, Dk, H = 128, 128, 16, 2
    gen = torch.Generator().manual_seed(5)
    qbuf = torch.randn(H, G, D, generator=gen).half().to(dev)
    bi = torch.full((D,), Dk + 1, dtype=torch.uint8)
    bi[torch.randperm(D, generator=gen)[:Dk]] = torch.arange(Dk, dtype=torch.uint8)
    bi = bi.to(dev)
    kb = torch.zeros(4, H, D, G // 4, dtype=torch.uint8, device=dev)
    kh = torch.zeros(4, H, Dk, G // 4, dtype=torch.uint8, device=dev)
    km = torch.zeros(4, H, 2, D, dtype=torch.float16, device=dev)
    vp = torch.zeros(4, H, G, D // 4, dtype=torch.uint8, device=dev)
    vm = torch.zeros(4, H, G, 2, dtype=torch.float16, device=dev)
    key_block = qbuf[1].T.contiguous()        # pipeline.py:219
    quantize_key_page(key_block, bi, Dk, Dk + 1, kb[2, 1], kh[2, 1], km[2, 1, 0], km[2, 1, 1])
    quantize_value_page(qbuf[0], vp[2, 1], vm[2, 1, :, 0], vm[2, 1, :, 1])   # strided scale/zero views
    t2b, th, s, z = quantize_key_page_torch(key_block, bi, Dk, Dk + 1)
    pk, sv, zv = quantize_value_page_torch(qbuf[0])
    torch.cuda.synchronize()
    e = O.quantize_key(key_block.cpu().numpy(), bi.cpu().numpy(), Dk, Dk + 1)
    ev = O.quantize_value(qbuf[0].cpu().numpy())
    assert np.array_equal(kb[2, 1].cpu().numpy(), e[0]) and np.array_equal(t2b.cpu().numpy(), e[0])
    assert np.array_equal(kh[2, 1].cpu().numpy(), e[1]) and np.array_equal(th.cpu().numpy(), e[1])
    assert _eq16(km[2, 1, 0].cpu(), e[2]) and _eq16(s.cpu(), e[2]) and _eq16(z.cpu(), e[3])
    assert np.array_equal(vp[2, 1].cpu().numpy(), ev[0]) and np.array_equal(pk.cpu().numpy(), ev[0])
    assert _eq16(vm[2, 1, :, 0].cpu(), ev[1]) and _eq16(vm[2, 1, :, 1].cpu(), ev[2]) and _eq16(zv.cpu(), ev[2])
    assert kb[[0, 1, 3]].sum() == 0 and kb[2, 0].sum() == 0      # nothing else written
    dk = dequantize_key_page_torch(t2b, th, s, z, bi, Dk)
    assert np.array_equal(dk.cpu().numpy(), O.dequantize_key(*e, bi.cpu().numpy(), Dk))
    dv = dequantize_value_page_torch(pk, sv, zv)
    assert np.array_equal(dv.cpu().numpy(), O.dequantize_value(*ev))
    out16 = torch.empty(D, G, dtype=torch.float16, device=dev)
    dequantize_key_page(t2b, th, s, z, bi, Dk, out16)
    assert np.array_equal(out16.cpu().numpy(), O.dequantize_key(*e, bi.cpu().numpy(), Dk).astype(np.float16))


def test_device_path_rejects_cpu_operands_and_matches_cpu_path(dev):
    """A device key with a CPU operand is refused by the HIP path (it never
    computes on the CPU); a CPU key runs the CPU path, whose bytes equal the
    kernel's."""
    from kitty.kernels import quantize_key_page_torch
    g = torch.Generator().manual_seed(8)
    key = (torch.randn(128, 128, generator=g) * 3).half()
    bi = torch.full((128,), 17, dtype=torch.uint8)
    bi[torch.randperm(128, generator=g)[:16]] = torch.arange(16, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="ROCm device"):
        quantize_key_page_torch(key.to(dev), bi, 16, 17)
    on_cpu = quantize_key_page_torch(key, bi, 16, 17)
    on_dev = quantize_key_page_torch(key.to(dev), bi.to(dev), 16, 17)
    assert all(a.device.type == "cpu" for a in on_cpu)
    for a, b in zip(on_cpu, on_dev):
        assert torch.equal(a, b.cpu())
