"""Host-side logic on CPU: KittyConfig derived constants and JSON round trip,
page pool shapes, first-fit free list, page table (re-expressing the
reference's tests/test_layout.py and tests/test_quantize.py:275-327)."""
import pytest
import torch

from kitty import KittyConfig, PageCentricKVLayoutManager


def _cfg(**kw):
    d = dict(num_layers=2, num_kv_heads=2, head_dim=16, q_buffer_size=8, sink_size=4, local_value_window=8,
             boost_rate=0.25, device="cpu")
    d.update(kw)
    return KittyConfig(**d)


def _layout(cfg):
    bi = torch.full((cfg.num_layers, cfg.num_kv_heads, cfg.head_dim), cfg.sentinel, dtype=torch.uint8)
    for i in range(cfg.d_boost):
        bi[:, :, i] = i
    return PageCentricKVLayoutManager(cfg, bi)


def test_derived_constants():
    c = KittyConfig()
    assert (c.d_boost, c.sentinel, c.max_pages) == (16, 17, 257)       # config.py:86-110
    p = KittyConfig.kitty_pro()
    assert (p.d_boost, p.sentinel, p.variant) == (32, 33, "kitty-pro")
    assert KittyConfig(boost_rate=0.5 / 128).d_boost == 0                # banker's rounding of 0.5
    with pytest.raises(AssertionError):
        KittyConfig(head_dim=30)
    with pytest.raises(AssertionError):
        KittyConfig(q_buffer_size=6)


def test_config_json_round_trip(tmp_path):
    c = _cfg(max_batch_size=4)
    c.save(tmp_path / "cfg.json")
    d = KittyConfig.load(tmp_path / "cfg.json")
    assert d == c
    import json
    assert "pool_pages_override" not in json.load(open(tmp_path / "cfg.json"))


def test_unique_physical_indices():
    lay = _layout(_cfg())
    phys = [lay.allocate_page(0, 0, i).physical_idx for i in range(5)]
    assert phys == [0, 1, 2, 3, 4]


def test_freed_slot_reused_first_fit():
    lay = _layout(_cfg())
    for i in range(4):
        lay.allocate_page(0, 0, i)
    lay.free_page(0, 0, 2)
    lay.free_page(0, 0, 0)
    assert lay.allocate_page(1, 0, 0).physical_idx == 0   # lowest free index first
    assert lay.allocate_page(1, 0, 1).physical_idx == 2
    assert lay.allocate_page(1, 0, 2).physical_idx == 4


def test_allocate_run_matches_page_by_page_first_fit():
    """allocate_run(count) takes the pages count allocate_page calls would,
    with the freed heap shorter than, as long as, and longer than the run
    (short runs pop the heap, long ones sort it and take its head), and
    records the same page table."""
    import random
    rng = random.Random(3)
    cfg = _cfg()
    a, b = _layout(cfg), _layout(cfg)
    live = []
    for step in range(200):
        if live and rng.random() < 0.45:
            for _ in range(rng.randint(1, 12)):
                if live:
                    seq, pno = live.pop(rng.randrange(len(live)))
                    a.free_page(seq, 0, pno)
                    b.free_page(seq, 0, pno)
            continue
        seq, count = step, rng.choice([1, 2, 3, 5, 9, 20])
        if count > a.memory_stats()["pages_free"]:
            continue
        run = a.allocate_run(seq, 0, 0, count)
        one = [b.allocate_page(seq, 0, j).physical_idx for j in range(count)]
        assert run == one, step
        live += [(seq, j) for j in range(count)]
    assert a._page_table == b._page_table and a._seq_keys == b._seq_keys
    assert a.memory_stats() == b.memory_stats()


def test_pool_exhaustion_raises():
    cfg = _cfg()
    lay = _layout(cfg)
    for i in range(cfg.max_pages):
        lay.allocate_page(0, 0, i)
    with pytest.raises(RuntimeError, match="exhausted"):
        lay.allocate_page(0, 0, cfg.max_pages)


def test_free_sequence_and_stats():
    lay = _layout(_cfg())
    for i in range(4):
        lay.allocate_page(7, 0, i)
    lay.allocate_page(8, 1, 0)
    assert lay.memory_stats()["pages_used"] == 5
    lay.free_sequence(7)
    s = lay.memory_stats()
    assert s["pages_used"] == 1 and s["pages_free"] == s["pages_total"] - 1
    with pytest.raises(KeyError):
        lay.get_physical_idx(7, 0, 0)
    assert lay.get_physical_idx(8, 1, 0) == 4


def test_pool_shapes_dtypes():
    cfg = _cfg()
    lay = _layout(cfg)
    P, H, D, G, K = cfg.max_pages, cfg.num_kv_heads, cfg.head_dim, cfg.q_buffer_size, cfg.d_boost
    assert lay.key_baseline.shape == (P, H, D, G // 4) and lay.key_baseline.dtype == torch.uint8
    assert lay.key_boost.shape == (P, H, K, G // 4)
    assert lay.key_metadata.shape == (P, H, 2, D) and lay.key_metadata.dtype == torch.float16
    assert lay.value_pool.shape == (P, H, G, D // 4)
    assert lay.value_metadata.shape == (P, H, G, 2)
    page = lay.allocate_page(0, 0, 0)
    assert lay.key_baseline_page(page.physical_idx).shape == (H, D, G // 4)
    assert lay.key_boost_page(page.physical_idx).shape == (H, K, G // 4)
    assert lay.key_meta_page(page.physical_idx).shape == (H, 2, D)
    assert lay.value_page(page.physical_idx).shape == (H, G, D // 4)
    assert lay.value_meta_page(page.physical_idx).shape == (H, G, 2)


def test_page_list_and_block_table():
    lay = _layout(_cfg())
    a = [lay.allocate_page(0, 0, i).physical_idx for i in range(3)]
    b = [lay.allocate_page(1, 0, i).physical_idx for i in range(1)]
    assert lay.get_page_list(0, 0) == a and lay.get_page_list(1, 0) == b
    bt, n, mx = lay.block_table([1, 0, 5], 0)
    assert bt.dtype == torch.int32 and bt.shape == (3, 3) and mx == 3
    assert bt[1].tolist() == a and bt[0, 0].item() == b[0] and n.tolist() == [1, 3, 0]


def test_pool_override_sizes_multi_layer_pools():
    cfg = _cfg(pool_pages_override=_cfg().max_pages * 2)
    lay = _layout(cfg)
    assert lay.key_baseline.shape[0] == cfg.max_pages * 2


def test_pipeline_counters_on_cpu():
    """Host bookkeeping and the CPU pipeline: sinks, buffers and a spill into
    a page on CPU pools (the spill's bytes are pinned in test_cpu_path.py)."""
    from kitty import KittyInferencePipeline
    cfg = _cfg(num_layers=1)
    lay = _layout(cfg)
    bi = torch.full((1, cfg.num_kv_heads, cfg.head_dim), cfg.sentinel, dtype=torch.uint8)
    p = KittyInferencePipeline(cfg, lay, bi)
    H, D = cfg.num_kv_heads, cfg.head_dim
    for _ in range(cfg.sink_size + 3):
        p.push_token(0, torch.randn(H, D).half(), torch.randn(H, D).half())
    assert p.sink_fill == cfg.sink_size and p.key_qbuf_len == 3 and p.val_local_len == 3
    ctx = p.get_attention_context(0)
    assert ctx["sink_k"].shape == (H, cfg.sink_size, D) and ctx["key_qbuf"].shape == (H, 3, D)
    for _ in range(cfg.q_buffer_size - 3):
        p.push_token(0, torch.randn(H, D).half(), torch.randn(H, D).half())
    assert p.key_qbuf_len == 0 and len(lay.get_page_list(0, 0)) == 1
    assert lay.key_metadata[lay.get_page_list(0, 0)[0], :, 0].abs().sum() > 0
