"""The pipeline's spill bookkeeping on the device: kitty_store_i32 (a list
of int32 stores carried in the kernel arguments) against indexed writes,
across the per-launch list limit; kitty_quant_batch's value_page_ids and
value_shift (keys and values of one spill into different pages, then the
value window's shift, in one launch) against separate launches and a torch
copy, on the production and the shape-generic kernel; and the pipeline's
spill of a single sequence and of sequences in lockstep against the staged,
indexed writes of its general path."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib():
    from kitty import _hip
    return _hip, _hip.load()


def test_store_i32_matches_indexed_writes(dev):
    _hip, L = _lib()
    rng = np.random.default_rng(5)
    for n in (1, 319, 320, 321, 1000):
        buf = torch.full((4096,), -7, dtype=torch.int32, device=dev)
        other = torch.full((64,), -9, dtype=torch.int32, device=dev)
        idx = rng.choice(4096, size=min(n, 4000), replace=False)
        vals = rng.integers(-2**31, 2**31 - 1, size=len(idx)).astype(np.int32)
        addrs = (buf.data_ptr() + 4 * idx).astype(np.int64)
        # one write into a second allocation in the same call
        addrs = np.append(addrs, other.data_ptr() + 4 * 17)
        vals = np.append(vals, np.int32(1234567))
        print(f"store_i32 n={len(addrs)}", flush=True)
        _hip.check(L.kitty_store_i32(addrs.ctypes.data, vals.ctypes.data, len(addrs), _hip.stream_ptr(dev)))
        want = torch.full((4096,), -7, dtype=torch.int32)
        want[torch.from_numpy(idx)] = torch.from_numpy(vals[:-1])
        assert torch.equal(buf.cpu(), want)
        assert int(other[17]) == 1234567 and int((other != -9).sum()) == 1


@pytest.mark.parametrize("D,G,R", [(128, 128, 128), (128, 128, 64), (64, 32, 32)])
def test_value_pages_and_shift_in_one_launch(dev, D, G, R):
    from kitty.kernels.ops import QuantizePlan, pool_store
    H, B, P = 2, 3, 16
    gen = torch.Generator(device=dev).manual_seed(D + G + R)
    pools = [torch.zeros(P, H, D, G // 4, dtype=torch.uint8, device=dev),
             torch.zeros(P, H, 4, G // 4, dtype=torch.uint8, device=dev),
             torch.zeros(P, H, 2, D, dtype=torch.float16, device=dev),
             torch.zeros(P, H, G, D // 4, dtype=torch.uint8, device=dev),
             torch.zeros(P, H, G, 2, dtype=torch.float16, device=dev)]
    twin = [t.clone() for t in pools]
    kbuf = torch.randn(B, H, G, D, device=dev, generator=gen).half()
    vbuf = torch.randn(B, H, R + G, D, device=dev, generator=gen).half()
    bi = torch.full((H, D), 5, dtype=torch.uint8, device=dev)
    bi[:, :4] = torch.arange(4, dtype=torch.uint8, device=dev)
    kp = torch.tensor([3, 9, 1], dtype=torch.int32, device=dev)
    vp = torch.tensor([12, 4, 7], dtype=torch.int32, device=dev)
    want_shift = vbuf.clone()
    want_shift[:, :, :R] = vbuf[:, :, G:G + R]
    v0 = vbuf.clone()
    # one launch: keys into kp, values into vp, then the shift
    print(f"value pages + shift D={D} G={G} R={R}", flush=True)
    QuantizePlan(pool_store(*pools), kbuf, vbuf[:, :, :G], bi, kp, 5, value_page_ids=vp, value_shift=R).run()
    # reference: separate launches on the twin pools from the unshifted values
    QuantizePlan(pool_store(*twin), kbuf, None, bi, kp, 5).run()
    QuantizePlan(pool_store(*twin), None, v0[:, :, :G], None, vp, 5).run()
    torch.cuda.synchronize()
    for a, b in zip(pools, twin):
        assert torch.equal(a, b)
    assert torch.equal(vbuf, want_shift)


def test_value_shift_rejects_rows_outside_the_storage(dev):
    from kitty.kernels.ops import QuantizePlan, pool_store
    pools = [torch.zeros(4, 1, 128, 32, dtype=torch.uint8, device=dev),
             torch.zeros(4, 1, 4, 32, dtype=torch.uint8, device=dev),
             torch.zeros(4, 1, 2, 128, dtype=torch.float16, device=dev),
             torch.zeros(4, 1, 128, 32, dtype=torch.uint8, device=dev),
             torch.zeros(4, 1, 128, 2, dtype=torch.float16, device=dev)]
    v = torch.zeros(1, 1, 128, 128, dtype=torch.float16, device=dev)     # no rows past G
    ids = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="outside"):
        QuantizePlan(pool_store(*pools), None, v, None, ids, 5, value_shift=64)


@pytest.mark.parametrize("ids", [[0], [0, 1, 2], [2, 0, 1]])
def test_spill_runs_match_general_path(dev, ids):
    """The same token stream through two pipelines, one spilling through the
    kernel-argument path (runs of slots) and one forced onto the staged,
    indexed path: pools, block tables, counters and value buffers equal
    after several key and value spills (R = 128, G = 128)."""
    from kitty import KittyConfig, KittyInferencePipeline, PageCentricKVLayoutManager
    import kitty.pipeline as P
    cfg = KittyConfig(num_layers=2, num_kv_heads=2, head_dim=128, q_buffer_size=128, sink_size=32,
                      local_value_window=128, boost_rate=0.125, max_seq_len=1024, max_batch_size=3, device="cuda:0")
    H, D = 2, 128
    bi = torch.full((2, H, D), cfg.sentinel, dtype=torch.uint8)
    for l in range(2):
        for h in range(H):
            bi[l, h, torch.randperm(D, generator=torch.Generator().manual_seed(10 * l + h))[:cfg.d_boost]] = \
                torch.arange(cfg.d_boost, dtype=torch.uint8)
    pipes = []
    for _ in range(2):
        lay = PageCentricKVLayoutManager(cfg, bi)
        pipes.append((KittyInferencePipeline(cfg, lay, bi), lay))
    fast, slow = pipes[0][0], pipes[1][0]
    slow._spill_runs = None          # never called: the run check below sends slow elsewhere
    orig = P._is_run
    gen = torch.Generator(device=dev).manual_seed(7)
    T = 32 + 3 * 128 + 140
    for t in range(T):
        for l in range(2):
            k = torch.randn(len(ids), H, D, device=dev, generator=gen).half()
            v = torch.randn(len(ids), H, D, device=dev, generator=gen).half()
            fast.push_tokens(l, k, v, ids)
            P._is_run = lambda s: False      # the staged path for every spill of `slow`
            try:
                slow.push_tokens(l, k, v, ids)
            finally:
                P._is_run = orig
    torch.cuda.synchronize()
    (la, lb) = pipes[0][1], pipes[1][1]
    for a, b in zip((la.key_baseline, la.key_boost, la.key_metadata, la.value_pool, la.value_metadata),
                    (lb.key_baseline, lb.key_boost, lb.key_metadata, lb.value_pool, lb.value_metadata)):
        assert torch.equal(a, b)
    assert torch.equal(fast._block_table, slow._block_table)
    assert torch.equal(fast.lens, slow.lens)
    assert torch.equal(fast._vbuf, slow._vbuf) and torch.equal(fast._qbuf_k, slow._qbuf_k)
    assert np.array_equal(fast._counts, slow._counts)
