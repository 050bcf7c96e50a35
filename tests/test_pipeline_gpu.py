"""Pipeline and drop-in module on the GPU.

* the reference's pipeline-state tests (tests/test_attention.py:57-126);
* page bytes after spills are the oracle quantisation of the same tokens
  (keys of every page, values of the pages older than the value window) and
  the FP16 value buffer holds the newest values;
* KittyPagedAttention decode end to end against the oracle computed from the
  raw token history (sinks, key pages, value pages, key and value tails
  derived independently from n, G and the window R), including BASELINE
  config 1 (B1, 8Q/8KV, d128, context 1024, outlier key channels).
"""
import numpy as np
import pytest
import torch

import oracle as O
from histref import close as _close, oracle_from_history as _oracle_from_history
from kvgen import calibrate_boost_idx, outlier_keys

pytestmark = pytest.mark.gpu


def _cfg(**kw):
    from kitty import KittyConfig
    d = dict(num_layers=1, num_kv_heads=2, head_dim=16, q_buffer_size=8, sink_size=4, local_value_window=8,
             boost_rate=0.25, device="cuda:0")
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


def _tok(H, D, gen):
    return torch.randn(H, D, generator=gen).half(), torch.randn(H, D, generator=gen).half()


def test_reference_pipeline_state(dev):
    cfg = _cfg()
    H, D, G, S = cfg.num_kv_heads, cfg.head_dim, cfg.q_buffer_size, cfg.sink_size
    gen = torch.Generator().manual_seed(0)
    p, lay, _ = _pipe(cfg)
    for _ in range(S):
        p.push_token(0, *_tok(H, D, gen))
    assert p.sink_fill == S and p.key_qbuf_len == 0           # test_attention.py:57-68
    for _ in range(3):
        p.push_token(0, *_tok(H, D, gen))
    assert p.key_qbuf_len == 3 and p.val_local_len == 3       # :70-84
    for _ in range(G - 3):
        p.push_token(0, *_tok(H, D, gen))
    assert p.key_qbuf_len == 0 and len(lay.get_page_list(0, 0)) == 1   # :86-99
    # the window (R = G = 8): values stay FP16 until they are R tokens old
    assert p.val_local_len == 8 and p.val_qbuf_len == 0
    for _ in range(4):
        p.push_token(0, *_tok(H, D, gen))
    assert p.val_local_len == 8 and p.val_qbuf_len == 4 and p.get_attention_context(0)["value_pages"] == 0
    for _ in range(2 * G - 4):
        p.push_token(0, *_tok(H, D, gen))
    assert len(lay.get_page_list(0, 0)) == 3                  # :115-126
    assert p.get_attention_context(0)["value_pages"] == 2 and p.val_local_len == 8 and p.val_qbuf_len == 0
    p.reset_sequence(0)
    assert p.sink_fill == 0 and p.key_qbuf_len == 0 and lay.memory_stats()["pages_used"] == 0  # :101-113


@pytest.mark.parametrize("extra,R", [((2, 1, 0), None), ((2, 0, 1), None), ((2, 0, 1), 0), ((1, 2, 2), 64),
                                     ((2, 0, 2), 64)])
def test_spilled_pages_are_bit_exact(dev, extra, R):
    """Pages of every spill bit-exact against the oracle.  Sequence i pushes
    S + extra[i] G (+5 for the first) tokens: spills of slots 0 and 1
    together (a run of slots, read through slice views), of slots 0 and 2
    (a gather), with the value window off (keys and values spill together)
    and at R = 64 (value spills of slots 1 and 2, and of 0 and 2)."""
    kw = {} if R is None else {"local_value_window": R}
    cfg = _cfg(num_layers=2, head_dim=128, q_buffer_size=128, sink_size=32, boost_rate=0.125, max_batch_size=3,
               **kw)
    L, H, D, G, S = cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, cfg.q_buffer_size, cfg.sink_size
    gen = torch.Generator().manual_seed(1)
    bi = torch.stack([torch.stack([torch.full((D,), cfg.sentinel, dtype=torch.uint8) for _ in range(H)])
                      for _ in range(L)])
    for l in range(L):
        for h in range(H):
            bi[l, h, torch.randperm(D, generator=gen)[:cfg.d_boost]] = torch.arange(cfg.d_boost, dtype=torch.uint8)
    p, lay, _ = _pipe(cfg, bi)
    n_tok = {s: S + e * G + (5 if s == 0 else 3 * (e == 0)) for s, e in enumerate(extra)}
    hist = {s: [] for s in n_tok}
    for t in range(max(n_tok.values())):
        ids = [s for s in n_tok if t < n_tok[s]]
        for l in range(L):
            k = torch.randn(len(ids), H, D, generator=gen).half()
            v = torch.randn(len(ids), H, D, generator=gen).half()
            p.push_tokens(l, k, v, ids)
            for i, s in enumerate(ids):
                hist[s].append((l, k[i], v[i]))
    torch.cuda.synchronize()
    kb, kh, km, vp, vm = [t.cpu().numpy() for t in (lay.key_baseline, lay.key_boost, lay.key_metadata,
                                                     lay.value_pool, lay.value_metadata)]
    R = cfg.local_value_window
    for s in n_tok:
        for l in range(L):
            toks = [(k, v) for (ll, k, v) in hist[s] if ll == l]
            pages = lay.get_page_list(s, l)
            n = n_tok[s] - S
            assert len(pages) == n // G
            npv = max(0, n - R) // G
            slot = p.slot(s)
            assert int(p._npv[slot, l]) == npv and int(p._vlen[slot, l]) == max(0, n) - npv * G
            # the FP16 value buffer: the values of tokens npv G .. n, oldest first
            vb = p._vbuf[slot, l, :, :max(0, n) - npv * G].cpu()
            want = [v for _, v in toks[S + npv * G:]]
            if want:
                assert torch.equal(vb, torch.stack(want).transpose(0, 1))
            for pi, ph in enumerate(pages):
                blk = toks[S + pi * G: S + (pi + 1) * G]
                K = torch.stack([k for k, _ in blk]).numpy()   # (G, H, D)
                V = torch.stack([v for _, v in blk]).numpy()
                for h in range(H):
                    e = O.quantize_key(K[:, h].T.copy(), bi[l, h].numpy(), cfg.d_boost, cfg.sentinel)
                    assert np.array_equal(kb[ph, h], e[0]) and np.array_equal(kh[ph, h], e[1])
                    assert np.array_equal(km[ph, h, 0].astype(np.float32), e[2].astype(np.float32))
                    assert np.array_equal(km[ph, h, 1].astype(np.float32), e[3].astype(np.float32))
                    if pi >= npv:
                        continue      # values still FP16 (in the window)
                    ev = O.quantize_value(V[:, h].copy())
                    assert np.array_equal(vp[ph, h], ev[0])
                    assert np.array_equal(vm[ph, h, :, 0].astype(np.float32), ev[1].astype(np.float32))


def test_config1_module_decode_step(dev):
    """one KittyPagedAttention decode step, B1, 8 Q / 8 KV
    heads, d128, context 1024 (32 sinks + 7 pages + 96 tail... + the new
    token), 12.5% INT4 channels from 256 calibration tokens with x8 outliers."""
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
    # prefill 1023 tokens, decode the 1024th
    q0 = torch.randn(1, Hq, 1023, D, generator=gen).half()
    attn(q0.to(dev), K[:1023].permute(1, 0, 2)[None].to(dev), V[:1023].permute(1, 0, 2)[None].to(dev))
    q = torch.randn(1, Hq, 1, D, generator=gen).half()
    out = attn(q.to(dev), K[1023:].permute(1, 0, 2)[None].to(dev), V[1023:].permute(1, 0, 2)[None].to(dev))
    assert out.shape == (1, Hq, 1, D) and out.dtype == torch.float16
    ref = _oracle_from_history(K.numpy(), V.numpy(), q[0, :, 0].numpy(), 32, 128, bi.numpy(), cfg.d_boost,
                               cfg.sentinel, Hq, H, D, R=128)
    _close(out[0, :, 0].cpu().numpy(), ref)


def test_batched_module_decode_gqa(dev):
    """Three sequences of different lengths decoded together through the
    module (GQA 4, MFMA path, 128-token value window: key pages run one
    ahead of value pages once a sequence passes 256 tokens), checked per
    sequence against the oracle.  The cached decode plan is reused across
    the steps and rebuilt when the batch changes."""
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
    steps = max(lens)
    for t in range(steps):
        ids = [s for s in range(3) if t < lens[s]]
        k = torch.randn(len(ids), H, 1, D, generator=gen).half()
        v = torch.randn(len(ids), H, 1, D, generator=gen).half()
        q = torch.randn(len(ids), Hq, 1, D, generator=gen).half()
        out = attn(q.to(dev), k.to(dev), v.to(dev), seq_id=ids)
        for i, s in enumerate(ids):
            hist[s].append((k[i, :, 0], v[i, :, 0]))
        if t in (39, 160, 299):  # last step of some sequence: check everyone in the batch
            for i, s in enumerate(ids):
                Kh = torch.stack([a for a, _ in hist[s]]).numpy()
                Vh = torch.stack([b for _, b in hist[s]]).numpy()
                ref = _oracle_from_history(Kh, Vh, q[i, :, 0].numpy(), 32, 128, bi[0].numpy(), cfg.d_boost,
                                           cfg.sentinel, Hq, H, D, R=128)
                _close(out[i, :, 0].cpu().numpy(), ref)


def test_random_module_sessions(dev):
    """Seeded random sessions through KittyPagedAttention: per case a shape
    (head_dim, G, sinks, value window R, KV heads, GQA group), sequences that
    start with a prefill chunk or with single tokens, then decode steps over
    random subsets of the unfinished sequences (spills of keys and of the
    value window at their own times); at random steps every sequence of the
    step is checked against the oracle rebuilt from its raw token history."""
    import random
    from kitty import KittyAttentionFactory
    shapes = [(16, 8, 4, 8, 60), (16, 8, 4, 5, 60), (16, 8, 0, 0, 50), (32, 16, 3, 16, 90),
              (128, 128, 32, 128, 420), (128, 128, 32, 128, 300)]
    for case, (D, G, S, R, maxlen) in enumerate(shapes):
        rnd = random.Random(400 + case)
        gen = torch.Generator().manual_seed(400 + case)
        H = rnd.choice([1, 2]) if D == 128 else rnd.choice([1, 2, 4])
        Hq = H * rnd.choice([1, 2, 4, 8])
        B = rnd.choice([2, 3, 4])
        cfg = _cfg(num_kv_heads=H, head_dim=D, q_buffer_size=G, sink_size=S, local_value_window=R,
                   boost_rate=0.125 if D == 128 else 0.25, max_seq_len=maxlen + 8, max_batch_size=B)
        bi = torch.full((1, H, D), cfg.sentinel, dtype=torch.uint8)
        for h in range(H):
            bi[0, h, torch.randperm(D, generator=gen)[:cfg.d_boost]] = torch.arange(cfg.d_boost, dtype=torch.uint8)
        layout, pipe, layers = KittyAttentionFactory.from_config(cfg, bi, Hq)
        attn = layers[0]
        lens = [rnd.randint(2, maxlen) for _ in range(B)]
        hist = [[] for _ in range(B)]
        # a prefill chunk of one length for a random subset of the sequences
        pre = [s for s in range(B) if rnd.random() < 0.5]
        if pre:
            T = rnd.randint(1, min(lens[s] for s in pre) - 1)
            k = torch.randn(len(pre), H, T, D, generator=gen).half()
            v = torch.randn(len(pre), H, T, D, generator=gen).half()
            q = torch.randn(len(pre), Hq, T, D, generator=gen).half()
            attn(q.to(dev), k.to(dev), v.to(dev), seq_id=pre)
            for i, s in enumerate(pre):
                hist[s].extend((k[i, :, t], v[i, :, t]) for t in range(T))
        checked = 0
        while any(len(hist[s]) < lens[s] for s in range(B)):
            live = [s for s in range(B) if len(hist[s]) < lens[s]]
            ids = sorted(rnd.sample(live, rnd.randint(1, len(live))))
            k = torch.randn(len(ids), H, 1, D, generator=gen).half()
            v = torch.randn(len(ids), H, 1, D, generator=gen).half()
            q = torch.randn(len(ids), Hq, 1, D, generator=gen).half()
            out = attn(q.to(dev), k.to(dev), v.to(dev), seq_id=ids)
            for i, s in enumerate(ids):
                hist[s].append((k[i, :, 0], v[i, :, 0]))
            if rnd.random() < 0.08 or all(len(hist[s]) >= lens[s] for s in range(B)):
                checked += 1
                for i, s in enumerate(ids):
                    Kh = torch.stack([a for a, _ in hist[s]]).numpy()
                    Vh = torch.stack([b for _, b in hist[s]]).numpy()
                    ref = _oracle_from_history(Kh, Vh, q[i, :, 0].numpy(), S, G, bi[0].numpy(), cfg.d_boost,
                                               cfg.sentinel, Hq, H, D, R=R)
                    _close(out[i, :, 0].cpu().numpy(), ref)
        assert checked > 0


def test_prefill_output_is_causal_attention(dev):
    from kitty import KittyAttentionFactory
    cfg = _cfg(num_kv_heads=2, head_dim=16, q_buffer_size=8, sink_size=4)
    gen = torch.Generator().manual_seed(13)
    layout, pipe, layers = KittyAttentionFactory.from_config(cfg, _boost(cfg), 4)
    q = torch.randn(1, 4, 21, 16, generator=gen).half()
    k = torch.randn(1, 2, 21, 16, generator=gen).half()
    v = torch.randn(1, 2, 21, 16, generator=gen).half()
    out = layers[0](q.to(dev), k.to(dev), v.to(dev)).float().cpu()
    ke, ve = k.float().repeat_interleave(2, 1), v.float().repeat_interleave(2, 1)
    s = (q.float() @ ke.transpose(-1, -2)) / 4.0
    s = s.masked_fill(torch.triu(torch.ones(21, 21, dtype=torch.bool), 1), float("-inf"))
    ref = torch.softmax(s, -1) @ ve
    assert torch.allclose(out, ref, atol=2e-3, rtol=1e-2)
    assert len(layout.get_page_list(0, 0)) == (21 - 4) // 8 and pipe.key_qbuf_len == (21 - 4) % 8


def _logical_pages(p, lay, seq, layer):
    """Page bytes of a sequence in logical order, from the five pools."""
    out = []
    for phys in lay.get_page_list(seq, layer):
        out.append(tuple(t[phys].cpu() for t in (lay.key_baseline, lay.key_boost, lay.key_metadata,
                                                  lay.value_pool, lay.value_metadata)))
    return out


@pytest.mark.parametrize("D,G,S,pre,T,R", [(16, 8, 4, 0, 61, 8), (16, 8, 4, 6, 50, 8), (16, 8, 4, 3, 70, 5),
                                           (16, 8, 4, 6, 50, 0), (128, 128, 32, 0, 700, 128),
                                           (128, 128, 32, 45, 400, 128), (128, 128, 32, 45, 400, 0)])
def test_bulk_prefill_matches_token_pushes(dev, D, G, S, pre, T, R):
    """push_chunk (bulk prefill: sinks and buffer rows copied, complete pages
    quantised straight from the chunk) leaves exactly the state of T single
    pushes: same sinks, key and value buffers, counters (host and device),
    page bytes; for value windows R = G, R = 0 (the single stream) and an R
    that is not a multiple of G."""
    cfg = _cfg(num_layers=2, num_kv_heads=2, head_dim=D, q_buffer_size=G, sink_size=S, local_value_window=R,
               boost_rate=0.125, max_batch_size=2)
    gen = torch.Generator().manual_seed(D + T)
    B, H = 2, cfg.num_kv_heads
    K = torch.randn(B, H, pre + T, D, generator=gen).half().to(dev)
    V = torch.randn(B, H, pre + T, D, generator=gen).half().to(dev)
    a, lay_a, _ = _pipe(cfg)
    b, lay_b, _ = _pipe(cfg)
    for layer in range(2):
        for t in range(pre):
            a.push_tokens(layer, K[:, :, t], V[:, :, t], [0, 1])
            b.push_tokens(layer, K[:, :, t], V[:, :, t], [0, 1])
        for t in range(pre, pre + T):
            a.push_tokens(layer, K[:, :, t], V[:, :, t], [0, 1])
        b.push_chunk(layer, K[:, :, pre:], V[:, :, pre:], [0, 1])
    torch.cuda.synchronize()
    for c in ("_fill", "_qlen", "_npages", "_npv", "_vlen"):
        assert np.array_equal(getattr(a, c), getattr(b, c)), c
    assert torch.equal(a.lens, b.lens)
    for i, c in enumerate(("_fill", "_qlen", "_npages", "_npv", "_vlen")):
        assert np.array_equal(a.lens[i].cpu().numpy().T, getattr(a, c)), c
    # the two streams cover the same tokens: (P_k - P_v) G + n_k = n_v
    assert np.array_equal((a._npages - a._npv) * G + a._qlen, a._vlen)
    for layer in range(2):
        for seq in range(B):
            s = a.slot(seq)
            f, q, v = int(a._fill[s, layer]), int(a._qlen[s, layer]), int(a._vlen[s, layer])
            assert torch.equal(a._sink_k[s, layer, :, :f], b._sink_k[s, layer, :, :f])
            assert torch.equal(a._sink_v[s, layer, :, :f], b._sink_v[s, layer, :, :f])
            assert torch.equal(a._qbuf_k[s, layer, :, :q], b._qbuf_k[s, layer, :, :q])
            assert torch.equal(a._vbuf[s, layer, :, :v], b._vbuf[s, layer, :, :v])
            pa, pb = _logical_pages(a, lay_a, seq, layer), _logical_pages(b, lay_b, seq, layer)
            assert len(pa) == len(pb) == int(a._npages[s, layer])
            for x, y in zip(pa, pb):
                assert all(torch.equal(u, v) for u, v in zip(x, y))
    assert not a.overflowed() and not b.overflowed()


def test_prefill_at_production_shape_is_bit_exact(dev):
    """push_chunk of 4,096 tokens for 16 new sequences (the bench's prefill
    shape: 8 KV heads x 128, 12.5 % INT4, S = 32, G = R = 128, outlier key
    channels x8): the pages are read in place from the prompt; 24 sampled
    (sequence, page) pairs, every head, bit-exact against the oracle (keys of
    every page, values of the 30 pages older than the window), the FP16 sinks
    and buffers equal to the prompt's rows, and the counters."""
    from kitty import KittyConfig, KittyInferencePipeline, PageCentricKVLayoutManager
    B, H, T, D, G, S, R = 16, 8, 4096, 128, 128, 32, 128
    cfg = KittyConfig(num_layers=1, num_kv_heads=H, head_dim=D, boost_rate=0.125, max_seq_len=T + 256,
                      max_batch_size=B, device="cuda:0")
    assert (cfg.sink_size, cfg.q_buffer_size, cfg.local_value_window) == (S, G, R)
    gen = torch.Generator().manual_seed(31)
    K, chans = outlier_keys(gen, (B, T), H, D, cfg.d_boost, 8.0)         # (B, T, H, D)
    calib, _ = outlier_keys(gen, (256,), H, D, cfg.d_boost, 8.0, channels=chans)
    bi = calibrate_boost_idx(calib, cfg.d_boost, cfg.sentinel)           # (H, D)
    Kd = K.permute(0, 2, 1, 3).contiguous().to(dev)                       # (B, H, T, D)
    Vd = torch.randn(B, H, T, D, generator=gen).half().to(dev)
    bid = bi[None].to(dev)
    lay = PageCentricKVLayoutManager(cfg, bid)
    pipe = KittyInferencePipeline(cfg, lay, bid)
    pipe.push_chunk(0, Kd, Vd, list(range(B)))
    torch.cuda.synchronize()
    n_k, n_v = (T - S) // G, (T - S - R) // G                            # 31 key pages, 30 value pages
    for c, want in (("_fill", S), ("_qlen", T - S - n_k * G), ("_npages", n_k), ("_npv", n_v),
                    ("_vlen", T - S - n_v * G)):
        assert (getattr(pipe, c)[:B, 0] == want).all(), c
    assert torch.equal(pipe.lens[:, 0, :B].cpu(), torch.from_numpy(pipe._counts[:, :B, 0]).int())
    Kc, Vc = Kd.cpu(), Vd.cpu()
    for s in (0, 7, 15):
        slot = pipe.slot(s)
        assert torch.equal(pipe._sink_k[slot, 0, :, :S].cpu(), Kc[s, :, :S])
        assert torch.equal(pipe._sink_v[slot, 0, :, :S].cpu(), Vc[s, :, :S])
        q, v = T - S - n_k * G, T - S - n_v * G
        assert torch.equal(pipe._qbuf_k[slot, 0, :, :q].cpu(), Kc[s, :, S + n_k * G:])
        assert torch.equal(pipe._vbuf[slot, 0, :, :v].cpu(), Vc[s, :, S + n_v * G:])
    kb, kh, km, vp, vm = (t.cpu().numpy() for t in (lay.key_baseline, lay.key_boost, lay.key_metadata,
                                                     lay.value_pool, lay.value_metadata))
    rng = np.random.default_rng(5)
    picks = [(int(b), int(p)) for b, p in zip(rng.integers(0, B, 22), rng.integers(0, n_k, 22))]
    picks += [(0, 0), (B - 1, n_k - 1)]
    for s, p in picks:
        ph = lay.get_page_list(s, 0)[p]
        t0 = S + p * G
        for h in range(H):
            e = O.quantize_key(Kc[s, h, t0:t0 + G].T.numpy().copy(), bi[h].numpy(), cfg.d_boost, cfg.sentinel)
            assert np.array_equal(kb[ph, h], e[0]) and np.array_equal(kh[ph, h], e[1]), (s, p, h)
            assert np.array_equal(km[ph, h, 0].view(np.uint16), e[2].view(np.uint16)), (s, p, h)
            assert np.array_equal(km[ph, h, 1].astype(np.float32), e[3].astype(np.float32)), (s, p, h)
            if p < n_v:
                ev = O.quantize_value(Vc[s, h, t0:t0 + G].numpy().copy())
                assert np.array_equal(vp[ph, h], ev[0]), (s, p, h)
                assert np.array_equal(vm[ph, h, :, 0].view(np.uint16), ev[1].view(np.uint16)), (s, p, h)


def test_spill_on_full_pool_raises_and_leaves_state_unchanged(dev):
    """A push whose spill needs more pages than the pool has free raises the
    reference's exhaustion error (layout.py:161-203) before any state
    changes: counters, buffers and the free count are as before, the token
    is not appended, and after another sequence is reset the same push
    goes through."""
    cfg = _cfg(num_kv_heads=2, head_dim=16, q_buffer_size=8, sink_size=4, local_value_window=8,
               max_batch_size=3, pool_pages_override=5)
    H, D, G, S = cfg.num_kv_heads, cfg.head_dim, cfg.q_buffer_size, cfg.sink_size
    gen = torch.Generator().manual_seed(21)
    p, lay, _ = _pipe(cfg)
    ids = [0, 1, 2]
    for _ in range(S + G - 1):                   # one token short of the first spill
        k, v = torch.randn(3, H, D, generator=gen).half(), torch.randn(3, H, D, generator=gen).half()
        p.push_tokens(0, k, v, ids)
    k, v = torch.randn(3, H, D, generator=gen).half(), torch.randn(3, H, D, generator=gen).half()
    p.push_tokens(0, k, v, ids)                  # 3 key spills: 3 of the 5 pages
    for _ in range(G - 1):
        k, v = torch.randn(3, H, D, generator=gen).half(), torch.randn(3, H, D, generator=gen).half()
        p.push_tokens(0, k, v, ids)
    assert lay.memory_stats()["pages_free"] == 2
    before = {c: getattr(p, c).copy() for c in ("_fill", "_qlen", "_npages", "_npv", "_vlen")}
    lens_before = p.lens.clone()
    k, v = torch.randn(3, H, D, generator=gen).half(), torch.randn(3, H, D, generator=gen).half()
    with pytest.raises(RuntimeError, match="exhausted"):
        p.push_tokens(0, k, v, ids)              # needs 3 pages, 2 free
    torch.cuda.synchronize()
    assert lay.memory_stats()["pages_free"] == 2
    for c, a in before.items():
        assert np.array_equal(getattr(p, c), a), c
    assert torch.equal(p.lens, lens_before)
    assert not p.overflowed()
    p.reset_sequence(2)                          # frees its page: 3 free
    p.push_tokens(0, k[:2], v[:2], [0, 1])       # two key spills (and two value spills) fit now
    torch.cuda.synchronize()
    assert lay.memory_stats()["pages_free"] == 1
    assert [int(x) for x in p._npages[[p.slot(0), p.slot(1)], 0]] == [2, 2]
    assert [int(x) for x in p._npv[[p.slot(0), p.slot(1)], 0]] == [1, 1]
    assert not p.overflowed()
