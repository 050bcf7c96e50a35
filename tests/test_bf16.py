"""KittyConfig(dtype="bfloat16") (reference kitty/config.py:76): bf16 token
buffers and bf16 metadata pools (layout.py:123-137, pipeline.py:83-106).

The reference computes every scale and zero point in fp32, stores it as fp16
(quantize_key.py:121-122, quantize_value.py:90) and copies that into the
pool's dtype (quantize_key.py:263-269, quantize_value.py:223-227), so a bf16
pool holds bf16(fp16(x)); dequantisation and attention read the bf16 values
as fp32 (dequantize_key.py:92-95, kernels/attention.py:148-170).

CPU pins of the oracle's bf16 path:
* fp32 -> bf16 rounding equals torch's .to(torch.bfloat16) (round to nearest
  even, overflow to inf, subnormals) on edge and random values;
* bf16 blocks whose values fp16 also holds quantise to the same codes as the
  fp16 path (the same fp32 values enter the same arithmetic), with the stored
  scale and zero point bf16(fp16(x)) of the fp16 path's: this ties the bf16
  quantiser to the fp16 oracle pinned by the reference's known answers.
GPU parity (bit-exact pages, attention within atol 2e-3 / rtol 1e-2 of the
oracle) for the batch quantiser, the dequantisers, the decode and the
module.
"""
import warnings

import numpy as np
import pytest
import torch

import oracle as O
from kvgen import calibrate_boost_idx, outlier_keys


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ CPU pins

def test_bf16_rounding_matches_torch():
    edge = np.array([0.0, -0.0, 1.0, 1.00390625, 1.0078125, 1.01171875, 65504.0, 65520.0, 3.3961e38, 3.3964e38,
                     -3.3e38, np.inf, -np.inf, 1e-40, -1e-40, 1.1754944e-38, 2 ** -133], np.float32)
    rng = np.random.default_rng(0)
    rnd = (rng.standard_normal(200000) * 10.0 ** rng.integers(-35, 35, 200000)).astype(np.float32)
    x = np.concatenate([edge, rnd])
    x = x[np.isfinite(x) | np.isinf(x)]
    assert np.array_equal(O.f32_to_bf16(x), _bf16_bits(torch.from_numpy(x)))
    assert np.array_equal(O.bf16_to_f32(O.f32_to_bf16(x)), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_bf16_quantize_reduces_to_the_fp16_path():
    gen = torch.Generator().manual_seed(5)
    D, G, dk = 64, 32, 8
    bi = np.full(D, dk + 1, np.uint8)
    bi[np.random.default_rng(1).permutation(D)[:dk]] = np.arange(dk)
    for scale in (1.0, 8.0, 300.0):
        k = (torch.randn(D, G, generator=gen) * scale).to(torch.bfloat16)
        assert torch.equal(k.half().to(torch.bfloat16), k)          # fp16 holds these bf16 values
        kf16 = k.half().numpy()
        t2b, th, s, z = O.quantize_key(kf16, bi, dk, dk + 1)        # fp16 C oracle
        b2b, bth, bs, bz = O.quantize_key_bf16(_bf16_bits(k), bi, dk, dk + 1)
        assert np.array_equal(t2b, b2b) and np.array_equal(th, bth)
        assert np.array_equal(bs, O.f32_to_bf16(s.astype(np.float32)))
        assert np.array_equal(bz, O.f32_to_bf16(z.astype(np.float32)))
        v = (torch.randn(G, D, generator=gen) * scale).to(torch.bfloat16)
        p, vs, vz = O.quantize_value(v.half().numpy())
        bp, bvs, bvz = O.quantize_value_bf16(_bf16_bits(v))
        assert np.array_equal(p, bp) and np.array_equal(bvs, O.meta_bf16(vs)) and np.array_equal(bvz, O.meta_bf16(vz))


def test_bf16_known_answer_and_double_rounding():
    # [0,1,2,3] per channel (tests/test_quantize.py:141-166): scale 1, zero 0 in bf16 too
    key = np.tile(np.array([0, 1, 2, 3], np.float32), (4, 1))
    t2b, _, s, z = O.quantize_key_bf16(O.f32_to_bf16(key), np.full(4, 255, np.uint8), 0, 255)
    assert (t2b == 0xE4).all() and (s == 0x3F80).all() and (z == 0).all()
    # the pool holds bf16(fp16(s)), not bf16(s): a boosted channel spanning
    # [-0.5546875, 3.7103891e-06] has s = rng / 15 whose fp16 rounding lands on
    # a bf16 tie (0x3D18 after both roundings, 0x3D17 rounded once)
    hi = float(O.bf16_to_f32(O.f32_to_bf16(np.float32(3.7103891372680664e-06)))[0])
    row = np.array([[-0.5546875, hi, 0.0, 0.0]], np.float32)
    _, _, s1, _ = O.quantize_key_bf16(O.f32_to_bf16(row), np.zeros(1, np.uint8), 1, 2)
    s_direct = O.f32_to_bf16(np.float32(np.float32(hi) - np.float32(-0.5546875)) / np.float32(15.0))
    assert s1[0] == 0x3D18 and s_direct == 0x3D17
    # a bf16 value fp16 cannot hold: 3.0e5 (above fp16's 65504) gives an inf fp16 scale
    big = np.tile(np.array([0.0, 3.0e5, 0.0, 3.0e5], np.float32), (2, 1))
    _, sb, _ = O.quantize_value_bf16(O.f32_to_bf16(big))
    assert (sb == 0x7F80).all()


# ----------------------------------------------------------------- GPU parity

def _bf16_pools(P, H, D, G, Dk, dev):
    from kitty.kernels.ops import pool_store
    kb = torch.full((P, H, D, G // 4), 0xAA, dtype=torch.uint8, device=dev)
    kh = torch.full((P, H, Dk, G // 4), 0x55, dtype=torch.uint8, device=dev)
    km = torch.full((P, H, 2, D), 7.0, dtype=torch.bfloat16, device=dev)
    vp = torch.full((P, H, G, D // 4), 0x33, dtype=torch.uint8, device=dev)
    vm = torch.full((P, H, G, 2), 7.0, dtype=torch.bfloat16, device=dev)
    return (kb, kh, km, vp, vm), pool_store(kb, kh, km, vp, vm)


@pytest.mark.gpu
def test_bf16_quantize_pack_bit_exact(dev):
    """bf16 K/V (x8 outlier key channels, values up to ~1e5 on some tokens,
    beyond fp16) into bf16 pools: codes and the bf16(fp16(x)) metadata
    bit-exact against the oracle, on the production shape and a small one."""
    from kitty.kernels.ops import quantize_into_pools
    for T, H, D, G, Dk in ((1024, 8, 128, 128, 16), (96, 2, 16, 8, 4)):
        gen = torch.Generator().manual_seed(T + D)
        sentinel = Dk + 1
        K, chans = outlier_keys(gen, (T,), H, D, max(Dk, 1), 8.0)
        K = (K.float() * (1 + torch.rand(T, H, D, generator=gen))).to(torch.bfloat16)
        V = torch.randn(T, H, D, generator=gen)
        V[5] *= 1.0e5                                      # a token fp16 could not hold
        V = V.to(torch.bfloat16)
        calib, _ = outlier_keys(gen, (64,), H, D, max(Dk, 1), 8.0, channels=chans)
        bi = calibrate_boost_idx(calib, Dk, sentinel)
        n = T // G
        pools, store = _bf16_pools(n + 3, H, D, G, Dk, dev)
        page_ids = torch.randperm(n + 3, generator=gen)[:n].to(torch.int32)
        kblk = K.to(dev).view(n, G, H, D).permute(0, 2, 1, 3)
        vblk = V.to(dev).view(n, G, H, D).permute(0, 2, 1, 3)
        quantize_into_pools(store, kblk, vblk, bi.to(dev), page_ids.to(dev), sentinel)
        torch.cuda.synchronize()
        kb, kh, km, vp, vm = [t.cpu() for t in pools]
        for g in range(n):
            p = int(page_ids[g])
            for h in range(H):
                t2b, th, s, z = O.quantize_key_bf16(_bf16_bits(K[g * G:(g + 1) * G, h].T.contiguous()),
                                                    bi[h].numpy(), Dk, sentinel)
                assert np.array_equal(kb[p, h].numpy(), t2b) and np.array_equal(kh[p, h].numpy(), th), (g, h)
                assert np.array_equal(_bf16_bits(km[p, h, 0]), s) and np.array_equal(_bf16_bits(km[p, h, 1]), z)
                pk, vs, vz = O.quantize_value_bf16(_bf16_bits(V[g * G:(g + 1) * G, h].contiguous()))
                assert np.array_equal(vp[p, h].numpy(), pk), (g, h)
                assert np.array_equal(_bf16_bits(vm[p, h, :, 0]), vs) and np.array_equal(_bf16_bits(vm[p, h, :, 1]), vz)


@pytest.mark.gpu
def test_bf16_dequantize_into_every_output_dtype(dev):
    from kitty.kernels import dequantize_key_page
    from kitty.kernels.quantize_value import dequantize_value_page_torch
    gen = torch.Generator().manual_seed(9)
    D, G, Dk = 128, 128, 16
    bi = torch.full((D,), Dk + 1, dtype=torch.uint8)
    bi[torch.randperm(D, generator=gen)[:Dk]] = torch.arange(Dk, dtype=torch.uint8)
    k = (torch.randn(D, G, generator=gen) * 4).to(torch.bfloat16)
    t2b, th, s, z = O.quantize_key_bf16(_bf16_bits(k), bi.numpy(), Dk, Dk + 1)
    sf, zf = O.bf16_to_f32(s), O.bf16_to_f32(z)
    ref = O.dequantize_key_np(t2b, th, sf, zf, bi.numpy(), Dk)
    args = [torch.from_numpy(t2b).to(dev), torch.from_numpy(th).to(dev),
            torch.from_numpy(sf).to(torch.bfloat16).to(dev), torch.from_numpy(zf).to(torch.bfloat16).to(dev),
            bi.to(dev), Dk]
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        out = torch.empty(D, G, dtype=dt, device=dev)
        dequantize_key_page(*args, out)
        assert torch.equal(out.cpu(), torch.from_numpy(ref).to(dt)), dt        # the fp32 result rounded once
    v = (torch.randn(G, D, generator=gen) * 3).to(torch.bfloat16)
    pk, vs, vz = O.quantize_value_bf16(_bf16_bits(v))
    got = dequantize_value_page_torch(torch.from_numpy(pk).to(dev),
                                      torch.from_numpy(O.bf16_to_f32(vs)).to(torch.bfloat16).to(dev),
                                      torch.from_numpy(O.bf16_to_f32(vz)).to(torch.bfloat16).to(dev))
    assert np.array_equal(got.cpu().numpy(), O.dequantize_value_np(pk, O.bf16_to_f32(vs), O.bf16_to_f32(vz)))


def _close(got, ref, what=""):
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    assert np.isfinite(got).all(), what
    excess = np.abs(got - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert (excess <= 0).all(), f"{what}: max |diff| {np.abs(got - ref).max():.3g}"


@pytest.mark.gpu
def test_bf16_batched_decode_matches_oracle(dev):
    """Batched decode at the production shape with bf16 q, sinks, tails and
    metadata pools (quantised on the device from bf16 K/V): the generic
    kernel runs (plan.kernel, with one warning) and matches the oracle."""
    from kitty.kernels.ops import DecodePlan, quantize_into_pools
    gen = torch.Generator().manual_seed(21)
    B, Hq, H, D, G, Dk, S = 3, 16, 4, 128, 128, 16, 32
    sentinel = Dk + 1
    n_pages, tails = [3, 0, 5], [17, 96, 0]
    K, chans = outlier_keys(gen, (sum(n_pages) * G,), H, D, Dk, 8.0)
    K = K.float().to(torch.bfloat16)
    V = torch.randn(sum(n_pages) * G, H, D, generator=gen).to(torch.bfloat16)
    calib, _ = outlier_keys(gen, (64,), H, D, Dk, 8.0, channels=chans)
    bi = calibrate_boost_idx(calib, Dk, sentinel)
    P = sum(n_pages) + 4
    pools, store = _bf16_pools(P, H, D, G, Dk, dev)
    perm = torch.randperm(P, generator=gen)[:sum(n_pages)].to(torch.int32)
    n = sum(n_pages)
    quantize_into_pools(store, K.to(dev).view(n, G, H, D).permute(0, 2, 1, 3),
                        V.to(dev).view(n, G, H, D).permute(0, 2, 1, 3), bi.to(dev), perm.to(dev), sentinel)
    bt = torch.zeros(B, max(n_pages), dtype=torch.int32)
    off = 0
    for b in range(B):
        bt[b, :n_pages[b]] = perm[off:off + n_pages[b]]
        off += n_pages[b]
    bf = torch.bfloat16
    q = torch.randn(B, Hq, D, generator=gen).to(bf)
    sk, sv = torch.randn(B, H, S, D, generator=gen).to(bf), torch.randn(B, H, S, D, generator=gen).to(bf)
    T = max(tails)
    tk, tv = torch.randn(B, H, T, D, generator=gen).to(bf), torch.randn(B, H, T, D, generator=gen).to(bf)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    kb, kh, km, vp, vm = pools
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        import kitty.kernels.ops as ops
        ops._warned_generic = False
        plan = DecodePlan(q.to(dev), bt.to(dev), i32(n_pages), kb, kh, km, vp, vm, bi.to(dev), sk.to(dev),
                          sv.to(dev), i32([S] * B), tk.to(dev), tv.to(dev), i32(tails))
    assert plan.kernel == "generic"
    assert any("bfloat16" in str(x.message) for x in w)
    out = plan.run().cpu().numpy()
    assert out.dtype == np.float16
    kbn, khn, vpn = kb.cpu().numpy(), kh.cpu().numpy(), vp.cpu().numpy()
    kmn, vmn = km.float().cpu().numpy(), vm.float().cpu().numpy()
    f = lambda t: t.float().numpy()
    for b in range(B):
        pages = bt[b, :n_pages[b]].numpy()
        ref = O.paged_attention_kv(f(q[b]), pages, pages, kbn, khn, kmn, vpn, vmn, bi.numpy(), Dk, f(sk[b]),
                                   f(sv[b]), f(tk[b, :, :tails[b]]), f(tv[b, :, :tails[b]]), Hq, H, D)
        _close(out[b], ref, f"b={b}")


@pytest.mark.gpu
def test_bf16_module_decode_and_profiler(dev):
    """KittyPagedAttention with dtype="bfloat16": a 600-token bf16 prompt
    (prefill), then decode steps through the 128-token value window, checked
    against the oracle rebuilt from the raw bf16 token history; and the
    profiler's |k| sums of bf16 keys against float64."""
    from kitty import KittyAttentionFactory, KittyConfig
    from kitty.sensitivity import _ChannelAccumulator
    cfg = KittyConfig(num_layers=1, num_kv_heads=2, head_dim=128, q_buffer_size=128, sink_size=32,
                      local_value_window=128, boost_rate=0.125, max_seq_len=2048, dtype="bfloat16", device="cuda:0")
    H, D, Hq, G, S, R = 2, 128, 8, 128, 32, 128
    gen = torch.Generator().manual_seed(31)
    T0, steps = 600, 3
    K, chans = outlier_keys(gen, (T0 + steps,), H, D, cfg.d_boost, 8.0)
    K = K.float().to(torch.bfloat16)
    V = torch.randn(T0 + steps, H, D, generator=gen).to(torch.bfloat16)
    acc = _ChannelAccumulator(H, D, dev)
    acc.update(K[None].permute(0, 2, 1, 3).to(dev))
    want = K.double().abs().sum(0).numpy()
    assert np.allclose(acc.sum_abs.cpu().numpy(), want, rtol=1e-5, atol=1e-3)
    bi = calibrate_boost_idx(K[:256].float(), cfg.d_boost, cfg.sentinel)
    layout, pipe, layers = KittyAttentionFactory.from_config(cfg, bi[None], Hq)
    assert layout.key_metadata.dtype == torch.bfloat16 and pipe.buffer_dtype == torch.bfloat16
    attn = layers[0]
    q0 = torch.randn(1, Hq, T0, D, generator=gen).to(torch.bfloat16)
    attn(q0.to(dev), K[:T0].permute(1, 0, 2)[None].to(dev), V[:T0].permute(1, 0, 2)[None].to(dev))
    for t in range(T0, T0 + steps):
        q = torch.randn(1, Hq, 1, D, generator=gen).to(torch.bfloat16)
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", RuntimeWarning)
            out = attn(q.to(dev), K[t:t + 1].permute(1, 0, 2)[None].to(dev), V[t:t + 1].permute(1, 0, 2)[None].to(dev))
        n = t + 1
        npg, npv = (n - S) // G, max(0, n - S - R) // G
        kb = np.zeros((npg, H, D, G // 4), np.uint8)
        kh = np.zeros((npg, H, cfg.d_boost, G // 4), np.uint8)
        km = np.zeros((npg, H, 2, D), np.float32)
        vp = np.zeros((npg, H, G, D // 4), np.uint8)
        vm = np.zeros((npg, H, G, 2), np.float32)
        for pi in range(npg):
            blk = slice(S + pi * G, S + (pi + 1) * G)
            for h in range(H):
                a, b_, s, z = O.quantize_key_bf16(_bf16_bits(K[blk, h].T.contiguous()), bi[h].numpy(), cfg.d_boost,
                                                  cfg.sentinel)
                kb[pi, h], kh[pi, h], km[pi, h, 0], km[pi, h, 1] = a, b_, O.bf16_to_f32(s), O.bf16_to_f32(z)
                pk, vs, vz = O.quantize_value_bf16(_bf16_bits(V[blk, h].contiguous()))
                vp[pi, h], vm[pi, h, :, 0], vm[pi, h, :, 1] = pk, O.bf16_to_f32(vs), O.bf16_to_f32(vz)
        f = lambda x: x.float().numpy().transpose(1, 0, 2).copy()
        ref = O.paged_attention_kv(q[0, :, 0].float().numpy(), np.arange(npg), np.arange(npv), kb, kh, km, vp, vm,
                                   bi.numpy(), cfg.d_boost, f(K[:S]), f(V[:S]), f(K[S + npg * G:n]),
                                   f(V[S + npv * G:n]), Hq, H, D)
        _close(out[0, :, 0].float().cpu().numpy(), ref, f"step {t}")


@pytest.mark.gpu
def test_decode_path_names_the_kernel(dev):
    """plan.kernel reports the MFMA kernel for the production fp16 shape and
    the generic one, with a RuntimeWarning, when a boost rank repeats."""
    from kitty.kernels.ops import DecodePlan
    import kitty.kernels.ops as ops
    from kvgen import random_pools
    gen = torch.Generator().manual_seed(41)
    B, Hq, H, D, G, Dk, S = 2, 8, 2, 128, 128, 16, 32
    bi = torch.full((H, D), Dk + 1, dtype=torch.uint8)
    for h in range(H):
        bi[h, :Dk] = torch.arange(Dk, dtype=torch.uint8)
    pools = [t.to(dev) for t in random_pools(gen, 6, H, D, G, Dk, bi)]
    bt = torch.tensor([[0, 1, 2], [3, 4, 5]], dtype=torch.int32, device=dev)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    q = torch.randn(B, Hq, D, generator=gen).half().to(dev)
    sk = torch.randn(B, H, S, D, generator=gen).half().to(dev)
    tk = torch.randn(B, H, 5, D, generator=gen).half().to(dev)

    def plan(b):
        return DecodePlan(q, bt, i32([3, 2]), *pools, b.to(dev), sk, sk, i32([S, S]), tk, tk, i32([5, 1]))
    assert plan(bi).kernel == "mfma"
    q_mha = q[:, :H].contiguous()                      # one query head per KV head: padded to groups of 4
    assert DecodePlan(q_mha, bt, i32([3, 2]), *pools, bi.to(dev), sk, sk, i32([S, S]), tk, tk,
                      i32([5, 1])).kernel == "mfma"
    dup = bi.clone()
    dup[0, Dk] = 3                                   # rank 3 twice in head 0
    ops._warned_generic = False
    with pytest.warns(RuntimeWarning, match="repeats a rank"):
        p = plan(dup)
    assert p.kernel == "generic"
