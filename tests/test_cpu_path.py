"""The package on CPU tensors (``kitty.kernels.cpu``), pinned to the oracle.

The reference runs everything on CPU tensors through its PyTorch code, and
its own test suite is CPU-only (tests/test_quantize.py, tests/test_attention.py);
BASELINE config 1 is a decode step "on the repo's PyTorch CPU fallback".
Here the same calls on CPU tensors run the package's vectorised torch code:

* quantised codes, high rows, scales and zero points bit-exact against the C
  oracle (quantize_key.py:38-124, quantize_value.py:38-90), including outlier
  channels, constant and all-zero rows, gapped, repeated and d_boost ranks,
  bf16 blocks, batches of blocks, blocks written into strided pool views;
* dequantisation exact against the oracle;
* decode within the north star's tolerance (atol 2e-3, rtol 1e-2) of the
  oracle's decode, for the reference signature and the batched plan with
  ragged, empty and independent value streams; bad page ids poison only
  their sequence;
* the pipeline's spilled pages bit-exact, and the module's decode step
  (config 1 in full, and a batch) against the oracle rebuilt from the token
  history;
* the reference's own CPU tests (round-trip bounds, known answers, pipeline
  counters, sink-only attention) through this package's public names.
"""
import numpy as np
import pytest
import torch

import oracle as O
from histref import close, oracle_from_history
from kvgen import calibrate_boost_idx, outlier_keys


def _ranks(D, d_boost, sentinel, gen, gaps=False, repeat=False, with_d_boost=False):
    bi = torch.full((D,), sentinel, dtype=torch.uint8)
    perm = torch.randperm(D, generator=gen)
    ranks = list(range(d_boost))
    if gaps:
        ranks = ranks[::2]
    if repeat:
        ranks = ranks + ranks[:3]
    if with_d_boost:
        ranks = ranks + [d_boost]
    for i, r in enumerate(ranks):
        bi[perm[i]] = r
    return bi


def _key_block(gen, D, G, outliers=4, factor=8.0):
    k = torch.randn(D, G, generator=gen)
    k[torch.randperm(D, generator=gen)[:outliers]] *= factor
    k[1] = 0.75              # constant channel
    k[2] = 0.0               # all-zero channel
    k[3, : G // 2] = -2.5    # two-valued channel
    return k.half()


@pytest.mark.parametrize("D,G,d_boost,kind", [(128, 128, 16, "plain"), (128, 128, 32, "plain"),
                                               (128, 128, 16, "gaps"), (128, 128, 16, "repeat"),
                                               (128, 128, 16, "rank_d_boost"), (16, 8, 4, "plain"),
                                               (64, 32, 0, "plain")])
def test_quantize_key_bit_exact(D, G, d_boost, kind):
    from kitty.kernels import dequantize_key_page_torch, quantize_key_page_torch
    gen = torch.Generator().manual_seed(D + G + d_boost)
    sentinel = min(d_boost + 1, 255)
    for trial in range(3):
        key = _key_block(gen, D, G)
        bi = _ranks(D, d_boost, sentinel, gen, gaps=kind == "gaps", repeat=kind == "repeat",
                    with_d_boost=kind == "rank_d_boost")
        got = quantize_key_page_torch(key, bi, d_boost, sentinel)
        exp = O.quantize_key(key.numpy(), bi.numpy(), d_boost, sentinel)
        for g, e in zip(got[:2], exp[:2]):
            assert np.array_equal(g.numpy(), e)
        for g, e in zip(got[2:], exp[2:]):
            assert g.dtype == torch.float16
            assert np.array_equal(g.numpy().astype(np.float32), e.astype(np.float32))
        deq = dequantize_key_page_torch(*got, bi, d_boost)
        assert np.array_equal(deq.numpy(), O.dequantize_key(*exp, bi.numpy(), d_boost))


def test_quantize_value_bit_exact():
    from kitty.kernels import dequantize_value_page_torch, quantize_value_page_torch
    gen = torch.Generator().manual_seed(5)
    for G, D in ((128, 128), (8, 16), (32, 64)):
        v = torch.randn(G, D, generator=gen) * 3
        v[0] = 3.0          # constant positive row: codes 3, stored scale 0
        v[1] = -1.5         # constant negative row: codes 0
        v[2] = 0.0
        v[3, 5] = 40.0      # one large element
        v = v.half()
        got = quantize_value_page_torch(v)
        exp = O.quantize_value(v.numpy())
        assert np.array_equal(got[0].numpy(), exp[0])
        for g, e in zip(got[1:], exp[1:]):
            assert np.array_equal(g.numpy().astype(np.float32), e.astype(np.float32))
        assert np.array_equal(dequantize_value_page_torch(*got).numpy(), O.dequantize_value(*exp))


def test_batched_blocks_match_single_blocks_and_bf16():
    """A batch of blocks in one call equals per-block oracle results; bf16
    blocks that fp16 also holds give the fp16 codes with bf16(fp16(x))
    metadata (the reference's copy_ into a bf16 pool)."""
    from kitty.kernels import cpu
    gen = torch.Generator().manual_seed(9)
    N, H, D, G, dk = 3, 2, 128, 128, 16
    keys = torch.stack([torch.stack([_key_block(gen, D, G) for _ in range(H)]) for _ in range(N)])   # (N,H,D,G)
    bi = torch.stack([_ranks(D, dk, dk + 1, gen) for _ in range(H)])
    t2b, th, s, z = cpu.quantize_key_blocks(keys, bi, dk, dk + 1)
    vals = torch.randn(N, H, G, D, generator=gen).half()
    vp, vs, vz = cpu.quantize_value_blocks(vals)
    for n in range(N):
        for h in range(H):
            e = O.quantize_key(keys[n, h].numpy(), bi[h].numpy(), dk, dk + 1)
            assert np.array_equal(t2b[n, h].numpy(), e[0]) and np.array_equal(th[n, h].numpy(), e[1])
            assert np.array_equal(s[n, h].numpy(), e[2]) and np.array_equal(z[n, h].numpy(), e[3])
            ev = O.quantize_value(vals[n, h].numpy())
            assert np.array_equal(vp[n, h].numpy(), ev[0]) and np.array_equal(vs[n, h].numpy(), ev[1])
    kb16 = keys.to(torch.bfloat16)
    ok = kb16.float() == keys.float()            # elements fp16 and bf16 both hold
    keys_b = torch.where(ok, keys.float(), torch.zeros(())).to(torch.bfloat16)
    t2b_b, th_b, s_b, z_b = cpu.quantize_key_blocks(keys_b, bi, dk, dk + 1)
    ref = cpu.quantize_key_blocks(keys_b.float().half(), bi, dk, dk + 1)
    assert torch.equal(t2b_b, ref[0]) and torch.equal(th_b, ref[1]) and torch.equal(s_b, ref[2])
    bits = s_b.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits, O.meta_bf16(ref[2].numpy()))


def test_quantize_into_strided_pool_views_and_partial_value_rows():
    """The reference launchers write into pool views (pipeline.py:209-250);
    value rows past val_qbuf_len are zero padding (:240-243)."""
    from kitty.kernels import quantize_key_page, quantize_value_page
    from kitty import KittyConfig, PageCentricKVLayoutManager
    cfg = KittyConfig(num_layers=1, num_kv_heads=2, head_dim=128, q_buffer_size=128, sink_size=4,
                      boost_rate=0.125, device="cpu")
    gen = torch.Generator().manual_seed(3)
    bi = torch.stack([_ranks(128, cfg.d_boost, cfg.sentinel, gen) for _ in range(2)])
    lay = PageCentricKVLayoutManager(cfg, bi[None])
    before = [t.clone() for t in (lay.key_baseline, lay.key_boost, lay.key_metadata, lay.value_pool,
                                  lay.value_metadata)]
    p, h = 3, 1
    key = _key_block(gen, 128, 128)
    quantize_key_page(key, bi[h], cfg.d_boost, cfg.sentinel, lay.key_baseline[p, h], lay.key_boost[p, h],
                      lay.key_metadata[p, h, 0], lay.key_metadata[p, h, 1])
    val = torch.randn(128, 128, generator=gen).half()
    val[37:] = 0
    quantize_value_page(val, lay.value_pool[p, h], lay.value_metadata[p, h, :, 0], lay.value_metadata[p, h, :, 1])
    e = O.quantize_key(key.numpy(), bi[h].numpy(), cfg.d_boost, cfg.sentinel)
    assert np.array_equal(lay.key_baseline[p, h].numpy(), e[0])
    assert np.array_equal(lay.key_boost[p, h].numpy(), e[1])
    assert np.array_equal(lay.key_metadata[p, h].numpy(), np.stack([e[2], e[3]]))
    ev = O.quantize_value(val.numpy())
    assert np.array_equal(lay.value_pool[p, h].numpy(), ev[0])
    assert np.array_equal(lay.value_metadata[p, h].numpy(), np.stack([ev[1], ev[2]], -1))
    after = (lay.key_baseline, lay.key_boost, lay.key_metadata, lay.value_pool, lay.value_metadata)
    for b, a in zip(before, after):     # nothing outside (p, h) was touched
        mask = torch.ones(a.shape[:2], dtype=torch.bool)
        mask[p, h] = False
        assert torch.equal(b[mask], a[mask])


def _pools(gen, P, H, D, G, dk, bi, rng):
    """Pools filled by the oracle's quantiser from random blocks (x8 outliers)."""
    kb = np.zeros((P, H, D, G // 4), np.uint8)
    kh = np.zeros((P, H, dk, G // 4), np.uint8)
    km = np.zeros((P, H, 2, D), np.float16)
    vp = np.zeros((P, H, G, D // 4), np.uint8)
    vm = np.zeros((P, H, G, 2), np.float16)
    for p in range(P):
        for h in range(H):
            kb[p, h], kh[p, h], km[p, h, 0], km[p, h, 1] = O.quantize_key(_key_block(gen, D, G).numpy(), bi[h],
                                                                           dk, dk + 1)
            vp[p, h], vm[p, h, :, 0], vm[p, h, :, 1] = O.quantize_value(
                rng.standard_normal((G, D)).astype(np.float16))
    return kb, kh, km, vp, vm


@pytest.mark.parametrize("Hq,H,n_pages,n_sink,n_tail", [(8, 2, 5, 32, 17), (4, 4, 3, 0, 0), (8, 2, 0, 7, 0),
                                                        (16, 2, 4, 32, 96)])
def test_paged_attention_reference_signature(Hq, H, n_pages, n_sink, n_tail):
    from kitty.kernels import paged_attention, paged_attention_reference
    gen = torch.Generator().manual_seed(Hq * 7 + n_pages)
    rng = np.random.default_rng(n_pages)
    D = G = 128
    dk = 16
    bi = np.stack([_ranks(D, dk, dk + 1, gen).numpy() for _ in range(H)])
    pools = _pools(gen, 6, H, D, G, dk, bi, rng)
    pages = list(rng.permutation(6)[:n_pages])
    q = rng.standard_normal((Hq, D)).astype(np.float16)
    sk, sv = (rng.standard_normal((H, n_sink, D)).astype(np.float16) for _ in range(2))
    tk, tv = (rng.standard_normal((H, n_tail, D)).astype(np.float16) for _ in range(2))
    ref = O.paged_attention(q, pages, *pools, bi, dk, sk, sv, tk, tv, Hq, H, D)
    t = torch.from_numpy
    for fn in (paged_attention, paged_attention_reference):
        out = fn(t(q), pages, *(t(x) for x in pools), t(bi), dk, t(sk), t(sv), t(tk), t(tv), Hq, H, D)
        assert out.shape == (Hq, D) and out.dtype == torch.float16
        if n_pages + n_sink + n_tail == 0:
            assert not out.any()
        else:
            close(out.numpy(), ref)


def test_random_decode_shapes_on_cpu():
    """The GPU suite's seeded random decode shapes (those up to 40 pages and
    nine sequences) through the CPU path against the oracle."""
    import random
    from test_decode_gpu import _batched_case, _oracle_batched, _random_shape, _run_batched
    cpu_dev, n = torch.device("cpu"), 0
    for k in range(40):
        rnd = random.Random(8000 + k)
        D, G, dk, H, Hq, B, S, ctx, pps = _random_shape(rnd)
        if max(ctx) > 40 * G or B > 9:
            continue
        c = _batched_case(cpu_dev, 8000 + k, B, Hq, H, D, G, dk, ctx, S=S)
        out = _run_batched(cpu_dev, c, pages_per_split=pps)
        for b in range(B):
            close(out[b], _oracle_batched(c, Hq, H, D, b))
        n += 1
    assert n >= 20


def test_paged_attention_unequal_tails_raise():
    from kitty.kernels import paged_attention
    H, D, G = 2, 16, 8
    z = torch.zeros
    with pytest.raises(RuntimeError):
        paged_attention(z(4, D, dtype=torch.float16), [], z(1, H, D, G // 4, dtype=torch.uint8),
                        z(1, H, 4, G // 4, dtype=torch.uint8), z(1, H, 2, D, dtype=torch.float16),
                        z(1, H, G, D // 4, dtype=torch.uint8), z(1, H, G, 2, dtype=torch.float16),
                        z(H, D, dtype=torch.uint8), 4, z(H, 0, D, dtype=torch.float16),
                        z(H, 0, D, dtype=torch.float16), z(H, 3, D, dtype=torch.float16),
                        z(H, 2, D, dtype=torch.float16), 4, H, D)


def test_batched_plan_ragged_value_streams_and_poison():
    """paged_attention_batched on CPU tensors: ragged page counts, a sequence
    with no pages, independent value streams (P_v = P_k, P_k - 1, P_k - 2, 0),
    a bad page id and a wrong value length that poison only their sequence."""
    from kitty.kernels import paged_attention_batched
    gen = torch.Generator().manual_seed(21)
    rng = np.random.default_rng(21)
    B, Hq, H, D, G, dk = 7, 8, 2, 128, 128, 16
    P, W = 12, 5
    bi = np.stack([_ranks(D, dk, dk + 1, gen).numpy() for _ in range(H)])
    pools = _pools(gen, P, H, D, G, dk, bi, rng)
    npk = np.array([5, 3, 0, 4, 2, 5, 1])
    npv = np.array([5, 2, 0, 2, 0, 5, 1])
    ns = np.array([32, 32, 9, 32, 32, 32, 0])
    ntk = np.array([17, 0, 0, 96, 5, 40, 3])
    ntv = (npk - npv) * G + ntk
    ntv[5] += 1                      # wrong value length: sequence 5 is NaN
    bt = np.stack([rng.permutation(P)[:W] for _ in range(B)]).astype(np.int32)
    bt[6, 0] = P + 3                 # page id outside the pool: sequence 6 is NaN
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    S, T, TV = 32, 96, 96 + 2 * G + 1
    sk, sv = (rng.standard_normal((B, H, S, D)).astype(np.float16) for _ in range(2))
    tk = rng.standard_normal((B, H, T, D)).astype(np.float16)
    tv = rng.standard_normal((B, H, TV, D)).astype(np.float16)
    t = torch.from_numpy
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32))
    out = paged_attention_batched(t(q), t(bt), i32(npk), *(t(x) for x in pools), t(bi), t(sk), t(sv), i32(ns),
                                  t(tk), t(tv), i32(ntk), num_pages_v=i32(npv), tail_len_v=i32(ntv))
    for b in range(B):
        if b in (5, 6):
            assert torch.isnan(out[b]).all()
            continue
        ref = O.paged_attention_kv(q[b], bt[b, :npk[b]], bt[b, :npv[b]], *pools, bi, dk,
                                   sk[b, :, :ns[b]], sv[b, :, :ns[b]], tk[b, :, :ntk[b]], tv[b, :, :ntv[b]],
                                   Hq, H, D)
        close(out[b].numpy(), ref)


def _cfg(**kw):
    from kitty import KittyConfig
    d = dict(num_layers=1, num_kv_heads=2, head_dim=16, q_buffer_size=8, sink_size=4, local_value_window=8,
             boost_rate=0.25, device="cpu")
    d.update(kw)
    return KittyConfig(**d)


def _boost(cfg):
    bi = torch.full((cfg.num_layers, cfg.num_kv_heads, cfg.head_dim), cfg.sentinel, dtype=torch.uint8)
    for i in range(cfg.d_boost):
        bi[:, :, i] = i
    return bi


def _pipe(cfg, bi=None):
    from kitty import KittyInferencePipeline, PageCentricKVLayoutManager
    bi = _boost(cfg) if bi is None else bi
    lay = PageCentricKVLayoutManager(cfg, bi)
    return KittyInferencePipeline(cfg, lay, bi), lay, bi


def test_reference_pipeline_tests_on_cpu():
    """tests/test_attention.py:57-215 of the reference, on this package's CPU
    path: counters, page counts, reset, and paged_attention_reference over
    the pipeline's context (output shape, dtype, finite, sink-only)."""
    from kitty.kernels.attention import paged_attention_reference
    cfg = _cfg()
    H, D, G, S = cfg.num_kv_heads, cfg.head_dim, cfg.q_buffer_size, cfg.sink_size
    torch.manual_seed(0)
    p, lay, bi = _pipe(cfg)
    for _ in range(S):
        p.push_token(0, torch.randn(H, D).half(), torch.randn(H, D).half())
    assert p.sink_fill == S and p.key_qbuf_len == 0
    ctx = p.get_attention_context(0, 0)
    assert len(ctx["page_list"]) == 0
    out = paged_attention_reference(torch.randn(H, D).half(), [], lay.key_baseline, lay.key_boost,
                                    lay.key_metadata, lay.value_pool, lay.value_metadata, bi[0], cfg.d_boost,
                                    ctx["sink_k"], ctx["sink_v"], ctx["key_qbuf"], ctx["val_local"], H, H, D)
    assert out.shape == (H, D) and torch.isfinite(out).all()
    for _ in range(3):
        p.push_token(0, torch.randn(H, D).half(), torch.randn(H, D).half())
    assert p.key_qbuf_len == 3 and p.val_local_len == 3
    for _ in range(G - 3):
        p.push_token(0, torch.randn(H, D).half(), torch.randn(H, D).half())
    assert p.key_qbuf_len == 0 and len(lay.get_page_list(0, 0)) == 1
    ctx = p.get_attention_context(0, 0)
    q = torch.randn(H, D, dtype=torch.float16)
    out = paged_attention_reference(q, ctx["page_list"], lay.key_baseline, lay.key_boost, lay.key_metadata,
                                    lay.value_pool, lay.value_metadata, bi[0], cfg.d_boost, ctx["sink_k"],
                                    ctx["sink_v"], ctx["key_qbuf"], ctx["val_local"], H, H, D)
    assert out.shape == (H, D) and out.dtype == torch.float16 and torch.isfinite(out).all()
    for _ in range(2 * G):
        p.push_token(0, torch.randn(H, D).half(), torch.randn(H, D).half())
    assert len(lay.get_page_list(0, 0)) == 3
    p.reset_sequence(0)
    assert p.sink_fill == 0 and p.key_qbuf_len == 0 and lay.memory_stats()["pages_used"] == 0


def test_reference_quantize_tests_on_cpu():
    """tests/test_quantize.py:56-268 of the reference on this package's CPU
    path: round-trip bounds for INT2, INT4 and values, shapes, the [0,1,2,3]
    known answer (byte 0xE4, scale 1, zero 0) and the constant-value token."""
    from kitty.kernels import (dequantize_key_page_torch, dequantize_value_page_torch, quantize_key_page_torch,
                               quantize_value_page_torch)
    torch.manual_seed(1)
    D, G = 16, 8
    key = torch.randn(D, G).half()
    none = torch.full((D,), 5, dtype=torch.uint8)
    rec = dequantize_key_page_torch(*quantize_key_page_torch(key, none, 4, 5), none, 4)
    assert (key - rec.half()).abs().max() < 0.35 * (key.max() - key.min())
    bi15 = torch.full((D,), 16, dtype=torch.uint8)
    bi15[:15] = torch.arange(15, dtype=torch.uint8)
    out = quantize_key_page_torch(key, bi15, 15, 16)
    assert out[0].shape == (D, G // 4) and out[1].shape == (15, G // 4)
    rec = dequantize_key_page_torch(*out, bi15, 15)
    assert (key[:15] - rec[:15].half()).abs().max() < 0.12 * (key[:15].max() - key[:15].min())
    k4 = torch.tensor([[0.0, 1.0, 2.0, 3.0]] * 4).half()
    t2b, th, s, z = quantize_key_page_torch(k4, torch.full((4,), 255, dtype=torch.uint8), 0, 255)
    assert (t2b == 0xE4).all() and (s == 1).all() and (z == 0).all() and th.shape == (0, 1)
    v = torch.randn(G, D).half()
    packed, vs, vz = quantize_value_page_torch(v)
    assert packed.shape == (G, D // 4) and packed.dtype == torch.uint8 and vs.shape == (G,)
    rec = dequantize_value_page_torch(packed, vs, vz)
    rng = v.float().max(1).values - v.float().min(1).values
    assert ((v.float() - rec).abs().max(1).values < 0.35 * rng + 1e-3).all()
    packed, vs, vz = quantize_value_page_torch(torch.full((G, D), 3.0).half())
    assert (packed == 0xFF).all() and (vs == 0).all()
    assert not dequantize_value_page_torch(packed, vs, vz).any()


@pytest.mark.parametrize("R", [0, 8])
def test_spilled_pages_bit_exact(R):
    """Pages written by the CPU pipeline equal the oracle's quantisation of
    the same tokens: keys of every page, values of the pages older than the
    window; the rest of the values stay in the FP16 buffer."""
    cfg = _cfg(local_value_window=R, max_seq_len=256)
    H, D, G, S = cfg.num_kv_heads, cfg.head_dim, cfg.q_buffer_size, cfg.sink_size
    gen = torch.Generator().manual_seed(4 + R)
    p, lay, bi = _pipe(cfg)
    n = S + 5 * G + 3
    K = torch.randn(n, H, D, generator=gen).half()
    V = torch.randn(n, H, D, generator=gen).half()
    for i in range(n):
        p.push_token(0, K[i], V[i])
    ctx = p.get_attention_context(0, 0)
    pages = ctx["page_list"]
    assert len(pages) == 5 and ctx["value_pages"] == (5 * G + 3 - R) // G
    for pi, ph in enumerate(pages):
        blk = slice(S + pi * G, S + (pi + 1) * G)
        for h in range(H):
            e = O.quantize_key(K[blk, h].T.contiguous().numpy(), bi[0, h].numpy(), cfg.d_boost, cfg.sentinel)
            assert np.array_equal(lay.key_baseline[ph, h].numpy(), e[0])
            assert np.array_equal(lay.key_boost[ph, h].numpy(), e[1])
            assert np.array_equal(lay.key_metadata[ph, h].numpy(), np.stack([e[2], e[3]]))
            if pi < ctx["value_pages"]:
                ev = O.quantize_value(V[blk, h].numpy())
                assert np.array_equal(lay.value_pool[ph, h].numpy(), ev[0])
                assert np.array_equal(lay.value_metadata[ph, h].numpy(), np.stack([ev[1], ev[2]], -1))
    nv = ctx["val_local"].shape[1]
    assert torch.equal(ctx["val_local"], V[n - nv:].transpose(0, 1))


def test_config1_module_decode_step_on_cpu():
    """BASELINE config 1 as it is defined, on CPU tensors: one
    KittyPagedAttention decode step, B1, 8 Q / 8 KV heads, d128, context
    1024 (the prompt's 1023 tokens prefilled, the 1024th decoded), 12.5 %
    INT4 channels from 256 calibration tokens with x8 outliers, S = 32,
    G = R = 128, against the oracle rebuilt from the token history."""
    from kitty import KittyAttentionFactory
    cfg = _cfg(num_kv_heads=8, head_dim=128, q_buffer_size=128, sink_size=32, local_value_window=128,
               boost_rate=0.125, max_seq_len=2048)
    H, D, Hq = 8, 128, 8
    gen = torch.Generator().manual_seed(11)
    K, chans = outlier_keys(gen, (1024,), H, D, 16, 8.0)
    V = torch.randn(1024, H, D, generator=gen).half()
    calib, _ = outlier_keys(gen, (256,), H, D, 16, 8.0, channels=chans)
    bi = calibrate_boost_idx(calib, cfg.d_boost, cfg.sentinel)
    layout, pipe, layers = KittyAttentionFactory.from_config(cfg, bi[None], Hq)
    attn = layers[0]
    q0 = torch.randn(1, Hq, 1023, D, generator=gen).half()
    attn(q0, K[:1023].permute(1, 0, 2)[None], V[:1023].permute(1, 0, 2)[None])
    q = torch.randn(1, Hq, 1, D, generator=gen).half()
    out = attn(q, K[1023:].permute(1, 0, 2)[None], V[1023:].permute(1, 0, 2)[None])
    assert out.shape == (1, Hq, 1, D) and out.dtype == torch.float16 and out.device.type == "cpu"
    ref = oracle_from_history(K.numpy(), V.numpy(), q[0, :, 0].numpy(), 32, 128, bi.numpy(), cfg.d_boost,
                              cfg.sentinel, Hq, H, D, R=128)
    close(out[0, :, 0].numpy(), ref)


def test_batched_module_decode_on_cpu():
    """Three sequences of different lengths decoded together through the
    module on CPU tensors (GQA 4, 128-token value window), each checked
    against the oracle at the last step of a sequence."""
    from kitty import KittyAttentionFactory
    cfg = _cfg(num_kv_heads=2, head_dim=128, q_buffer_size=128, sink_size=32, boost_rate=0.125,
               local_value_window=128, max_seq_len=1024, max_batch_size=3)
    H, D, Hq = 2, 128, 8
    gen = torch.Generator().manual_seed(12)
    bi = torch.full((1, H, D), cfg.sentinel, dtype=torch.uint8)
    for h in range(H):
        bi[0, h, torch.randperm(D, generator=gen)[:cfg.d_boost]] = torch.arange(cfg.d_boost, dtype=torch.uint8)
    layout, pipe, layers = KittyAttentionFactory.from_config(cfg, bi, Hq)
    attn = layers[0]
    lens = [300, 161, 40]
    hist = [[], [], []]
    for t in range(max(lens)):
        ids = [s for s in range(3) if t < lens[s]]
        k = torch.randn(len(ids), H, 1, D, generator=gen).half()
        v = torch.randn(len(ids), H, 1, D, generator=gen).half()
        q = torch.randn(len(ids), Hq, 1, D, generator=gen).half()
        out = attn(q, k, v, seq_id=ids)
        for i, s in enumerate(ids):
            hist[s].append((k[i, :, 0], v[i, :, 0]))
        if t in (39, 160, 299):
            for i, s in enumerate(ids):
                Kh = torch.stack([a for a, _ in hist[s]]).numpy()
                Vh = torch.stack([b for _, b in hist[s]]).numpy()
                ref = oracle_from_history(Kh, Vh, q[i, :, 0].numpy(), 32, 128, bi[0].numpy(), cfg.d_boost,
                                          cfg.sentinel, Hq, H, D, R=128)
                close(out[i, :, 0].numpy(), ref)


def test_push_chunk_on_full_pool_leaves_batch_untouched():
    """push_chunk for sequences that already hold tokens allocates every
    sequence's pages before it changes any state: a full pool raises and
    the whole batch keeps its previous state."""
    cfg = _cfg(max_batch_size=3, max_seq_len=64, local_value_window=0)
    cfg.pool_pages_override = 6
    H, D, G, S = cfg.num_kv_heads, cfg.head_dim, cfg.q_buffer_size, cfg.sink_size
    p, lay, _ = _pipe(cfg)
    gen = torch.Generator().manual_seed(2)
    for s in range(3):                                   # each holds sinks + 1 page + 2 buffered keys
        for _ in range(S + G + 2):
            p.push_token(0, *(torch.randn(H, D, generator=gen).half() for _ in range(2)), seq_id=s)
    state = (p._counts.copy(), lay.memory_stats()["pages_used"], p._qbuf_k.clone(), lay.key_baseline.clone())
    chunk = torch.randn(3, H, 2 * G, D, generator=gen).half()   # two more pages each: 6 > 3 free
    with pytest.raises(RuntimeError, match="exhausted"):
        p.push_chunk(0, chunk, chunk, [0, 1, 2])
    assert np.array_equal(p._counts, state[0]) and lay.memory_stats()["pages_used"] == state[1]
    assert torch.equal(p._qbuf_k, state[2]) and torch.equal(lay.key_baseline, state[3])
    p.push_chunk(0, chunk[:1], chunk[:1], [0])           # room for one sequence's pages
    assert int(p._npages[p.slot(0), 0]) == 3
