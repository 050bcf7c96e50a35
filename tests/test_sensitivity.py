"""Channel-sensitivity profiler (reference kitty/sensitivity.py): ranking,
on-disk formats, and the device accumulation kernel."""
import json

import numpy as np
import pytest
import torch

from kitty import KittyConfig, KittySensitivityProfiler
from kitty.sensitivity import rank_channels


def test_rank_channels_known_answer():
    scores = torch.tensor([[[0.1, 5.0, 3.0, 5.0, 0.2, 4.0, 1.0, 2.0]]])   # (1, 1, 8); channels 1 and 3 tie
    masks, idx = rank_channels(scores, 3, 4)
    assert idx[0, 0].tolist() == [4, 0, 4, 1, 4, 2, 4, 4]                 # ties rank by channel index
    assert masks[0, 0].tolist() == [False, True, False, True, False, True, False, False]
    _, idx0 = rank_channels(scores, 0, 1)
    assert (idx0 == 1).all()


def test_rank_channels_matches_topk_without_ties():
    g = torch.Generator().manual_seed(1)
    scores = torch.rand(3, 4, 128, generator=g)
    masks, idx = rank_channels(scores, 16, 17)
    top = scores.topk(16, dim=-1).indices                                  # sensitivity.py:191-193
    ref = torch.zeros_like(masks).scatter_(-1, top, True)
    assert torch.equal(masks, ref)
    order = scores.argsort(dim=-1, descending=True)
    for r in range(16):                                                    # :197-203
        assert (idx.gather(-1, order[..., r:r + 1]) == r).all()


def test_save_load_formats(tmp_path):
    cfg = KittyConfig(num_layers=2, num_kv_heads=2, head_dim=16, boost_rate=0.25, device="cpu")
    prof = KittySensitivityProfiler(cfg)
    prof.scores_ = torch.rand(2, 2, 16, generator=torch.Generator().manual_seed(2))
    prof.boost_masks_, prof.boost_idx_uint8_ = rank_channels(prof.scores_, cfg.d_boost, cfg.sentinel)
    prof.save(tmp_path)
    for name, dtype in (("scores.pt", torch.float32), ("boost_masks.pt", torch.bool), ("boost_idx.pt", torch.uint8)):
        t = torch.load(tmp_path / name, weights_only=True)
        assert t.dtype == dtype and tuple(t.shape) == (2, 2, 16)
    meta = json.load(open(tmp_path / "meta.json"))
    assert meta["d_boost"] == cfg.d_boost and meta["head_dim"] == 16 and "token_count" in meta
    back = KittySensitivityProfiler.load(tmp_path, cfg)
    assert torch.equal(back.boost_idx_uint8, prof.boost_idx_uint8) and torch.equal(back.scores_, prof.scores_)


def test_summary_lines():
    cfg = KittyConfig(num_layers=2, num_kv_heads=2, head_dim=16, boost_rate=0.25, device="cpu")
    prof = KittySensitivityProfiler(cfg)
    assert prof.summary() == "KittySensitivityProfiler — not yet computed."
    prof.scores_ = torch.tensor([0.5, 1.5, 4.0, 2.0]).reshape(1, 1, 4).expand(2, 2, 4).contiguous()
    lines = prof.summary().split("\n")
    assert lines[0] == "KittySensitivityProfiler Summary"
    assert lines[1] == "  Layers: 2, KV Heads: 2, Head Dim: 16"
    assert lines[2] == "  Boost rate: 25.0% → 4 INT4 channels/head"
    assert lines[3] == "  Sentinel value: 5"
    assert lines[4] == "  Max channel score: 4.0000"
    assert lines[5] == "  Mean channel score: 2.0000"


def test_accumulation_on_cpu_matches_float64():
    """CPU keys are summed per (head, channel) over batch and tokens: the
    same scores as float64 sums, then the same ranking."""
    cfg = KittyConfig(num_layers=1, num_kv_heads=2, head_dim=16, device="cpu")
    prof = KittySensitivityProfiler(cfg)
    g = torch.Generator().manual_seed(6)
    keys = [torch.randn(2, 2, 9, 16, generator=g).half() for _ in range(3)]
    keys[1][:, :, :, 4] *= 16
    for k in keys:
        prof.update(0, k)
    ref = sum(k.double().abs().sum(dim=(0, 2)) for k in keys) / (3 * 2 * 9)
    assert torch.allclose(prof.accumulator(0).scores().double(), ref, rtol=1e-6)
    prof.compute()
    assert (prof.boost_idx_uint8[0, :, 4] == 0).all()


@pytest.mark.gpu
def test_abs_sum_kernel_matches_float64(dev):
    cfg = KittyConfig(num_layers=1, num_kv_heads=4, head_dim=128, device="cuda:0")
    g = torch.Generator().manual_seed(3)
    raw = torch.randn(3, 777, 4 * 128, generator=g)
    raw[..., 5] *= 8
    out = raw.half().to(dev)
    key = out.reshape(3, 777, 4, 128).permute(0, 2, 1, 3)                  # the hook's strided view
    prof = KittySensitivityProfiler(cfg)
    prof.update(0, key)
    prof.update(0, key[:1])
    acc = prof.accumulator(0)
    ref = np.abs(out.reshape(3, 777, 4, 128).cpu().double().numpy()).sum(axis=(0, 1))
    ref += np.abs(out[:1].reshape(1, 777, 4, 128).cpu().double().numpy()).sum(axis=(0, 1))
    np.testing.assert_allclose(acc.sum_abs.cpu().numpy(), ref, rtol=1e-5)
    assert acc.token_count == 4 * 777
    again = KittySensitivityProfiler(cfg)
    again.update(0, key)
    again.update(0, key[:1])
    assert torch.equal(again.accumulator(0).sum_abs, acc.sum_abs)          # fixed summation order


@pytest.mark.gpu
def test_hooks_on_key_projections(dev):
    H, D, L = 2, 64, 2

    class Attn(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.k_proj = torch.nn.Linear(32, H * D, bias=False)

    class Layer(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.self_attn = Attn()

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = torch.nn.ModuleList([Layer() for _ in range(L)])

        def forward(self, x):
            return [layer.self_attn.k_proj(x) for layer in self.layers]

    torch.manual_seed(4)
    model = Model().half().to(dev)
    cfg = KittyConfig(num_layers=L, num_kv_heads=H, head_dim=D, boost_rate=0.125, device="cuda:0")
    prof = KittySensitivityProfiler(cfg, model)
    prof.register_hooks(range(L))
    xs = [torch.randn(2, 50, 32, device=dev).half() for _ in range(3)]
    outs = [model(x) for x in xs]
    prof.remove_hooks()
    prof.compute()
    for l in range(L):
        k = torch.cat([o[l].float().reshape(-1, H, D) for o in outs])
        ref = k.abs().mean(0).cpu()
        torch.testing.assert_close(prof.scores_[l], ref, rtol=1e-4, atol=1e-6)
    _, want = rank_channels(prof.scores_, cfg.d_boost, cfg.sentinel)
    assert torch.equal(prof.boost_idx_uint8, want)


@pytest.mark.gpu
@pytest.mark.parametrize("B,T,H,D,how", [
    (50, 3, 2, 128, "two-pass"),     # 16 rows per step wrap several batch rows at once
    (2, 1000, 3, 64, "two-pass"),    # 8 lanes per row, 32 rows per step
    (1, 300, 2, 256, "two-pass"),    # 32 lanes per row, 8 rows per step
    (3, 12000, 2, 128, "two-pass"),  # more tokens than 256 chunks of one round: two rounds per chunk
    (2, 100, 2, 48, "fallback"),     # 6 lanes per row do not tile 256 threads
    (2, 100, 2, 128, "misaligned"),  # rows not 16-byte aligned
    (3, 200, 2, 128, "no-workspace"),
])
def test_abs_sum_paths(dev, B, T, H, D, how):
    """kitty_channel_abs_sum through each of its paths against float64, and
    the same bits on a repeated call (fixed summation order)."""
    import ctypes
    from kitty import _hip
    g = torch.Generator().manual_seed(B * T + D)
    raw = (torch.randn(B, H, T + 1, D, generator=g) * 3).half()
    key = raw[:, :, 1:] if how == "misaligned" else raw[:, :, :T]
    kd = raw.to(dev)[:, :, 1:] if how == "misaligned" else raw.to(dev)[:, :, :T]
    L = _hip.load()
    need = ctypes.c_size_t(0)
    _hip.check(L.kitty_channel_abs_sum_workspace_size(B, T, H, D, ctypes.byref(need)))
    assert (need.value > 0) == (how in ("two-pass", "misaligned", "no-workspace"))
    ws = torch.empty(max(need.value, 16), dtype=torch.uint8, device=dev)
    outs = []
    for _ in range(2):
        out = torch.zeros(H, D, dtype=torch.float32, device=dev)
        wp = None if how == "no-workspace" else ws.data_ptr()
        _hip.check(L.kitty_channel_abs_sum(kd.data_ptr(), kd.stride(0), kd.stride(2), kd.stride(1), B, T, H, D,
                                           _hip.KITTY_DTYPE_F16, out.data_ptr(), wp, need.value,
                                           _hip.stream_ptr(torch.device(dev))))
        torch.cuda.synchronize()
        outs.append(out.cpu())
    want = key.double().abs().sum(dim=(0, 2)).numpy()
    np.testing.assert_allclose(outs[0].numpy(), want, rtol=1e-5)
    assert torch.equal(outs[0], outs[1])


@pytest.mark.gpu
def test_deferred_abs_sum_matches_float64_and_repeats():
    """kitty_channel_abs_sum_deferred over updates of different shapes (one
    more than 256 chunks of one round, one misaligned by an element, which
    adds into out at once), with a flush in the middle and at the end: the
    float64 sum, the same bits on a second run of the same calls, zeroed
    slots, and a flush with nothing pending adds nothing."""
    import ctypes
    from kitty import _hip
    L = _hip.load()
    H, D = 3, 128
    need = ctypes.c_size_t(0)
    _hip.check(L.kitty_channel_abs_sum_deferred_size(H, D, ctypes.byref(need)))
    assert need.value == H * D * 256 * 4
    g = torch.Generator().manual_seed(77)
    shapes = ((2, 700, False), (5, 3, False), (3, 12000, False), (1, 300, True))
    keys = [(torch.randn(B, H, T, D, generator=g) * 2).half() for B, T, _ in shapes]

    def run():
        slots = torch.zeros(need.value, dtype=torch.uint8, device="cuda")
        out = torch.zeros(H, D, dtype=torch.float32, device="cuda")
        held = []
        for n, ((B, T, off), k) in enumerate(zip(shapes, keys)):
            flat = torch.empty(k.numel() + 1, dtype=torch.float16, device="cuda")
            flat[int(off):int(off) + k.numel()] = k.flatten().cuda()
            key = flat[int(off):int(off) + k.numel()].view(B, H, T, D)      # off: 2 bytes from 16-byte alignment
            held.append(flat)
            _hip.check(L.kitty_channel_abs_sum_deferred(key.data_ptr(), key.stride(0), key.stride(2), key.stride(1),
                                                        B, T, H, D, _hip.KITTY_DTYPE_F16, out.data_ptr(),
                                                        slots.data_ptr(), need.value, None))
            if n == 1:
                _hip.check(L.kitty_channel_abs_sum_flush(slots.data_ptr(), H, D, out.data_ptr(), None))
        _hip.check(L.kitty_channel_abs_sum_flush(slots.data_ptr(), H, D, out.data_ptr(), None))
        first = out.clone()
        _hip.check(L.kitty_channel_abs_sum_flush(slots.data_ptr(), H, D, out.data_ptr(), None))
        torch.cuda.synchronize()
        assert torch.equal(out, first) and slots.count_nonzero() == 0
        return out.cpu()

    a, b = run(), run()
    ref = sum(k.double().abs().sum(dim=(0, 2)) for k in keys)
    np.testing.assert_allclose(a.double().numpy(), ref.numpy(), rtol=1e-5)
    assert torch.equal(a, b)


def test_abs_sum_workspace_rejects_small_buffers():
    """A workspace below kitty_channel_abs_sum_workspace_size is refused
    before any device work (the pointers are never dereferenced)."""
    import ctypes
    from kitty import _hip
    L = _hip.load()
    need = ctypes.c_size_t(0)
    _hip.check(L.kitty_channel_abs_sum_workspace_size(4, 4096, 8, 128, ctypes.byref(need)))
    assert need.value == 8 * 128 * 128 * 4          # 4 x 4096 tokens per head: 128 chunks of 128
    fake = 1 << 20
    rc = L.kitty_channel_abs_sum(fake, 8 * 4096 * 128, 128, 4096 * 128, 4, 4096, 8, 128, _hip.KITTY_DTYPE_F16,
                                 fake, fake, need.value - 4, None)
    assert rc == _hip.KITTY_E_INVALID and b"workspace too small" in L.kitty_last_error()
    _hip.check(L.kitty_channel_abs_sum_deferred_size(8, 128, ctypes.byref(need)))
    assert need.value == 8 * 128 * 256 * 4                 # 256 slots per (head, channel), any batch
    rc = L.kitty_channel_abs_sum_deferred(fake, 8 * 4096 * 128, 128, 4096 * 128, 4, 4096, 8, 128,
                                          _hip.KITTY_DTYPE_F16, fake, fake, need.value - 4, None)
    assert rc == _hip.KITTY_E_INVALID and b"slot buffer too small" in L.kitty_last_error()
    _hip.check(L.kitty_channel_abs_sum_deferred_size(8, 48, ctypes.byref(need)))
    assert need.value == 0                                 # no 16-byte rows: deferred calls add at once
    assert L.kitty_channel_abs_sum_flush(None, 8, 48, None, None) == 0
