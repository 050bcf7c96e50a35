"""Committed golden fixtures (tests/golden/, written by make_golden.py):
the CPU oracle must reproduce them, and so must the HIP kernels on the GPU
(packed bytes and fp16 metadata bit-exact, attention within atol 2e-3 /
rtol 1e-2)."""
import os

import numpy as np
import pytest
import torch

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return dict(np.load(os.path.join(GOLD, name), allow_pickle=False))


def _bits(a):
    return np.ascontiguousarray(a, np.float16).view(np.uint16)


def test_oracle_reproduces_known_answers():
    g = _load("known_answers.npz")
    for fn in (O.quantize_key, O.quantize_key_np):
        t2b, th, s, z = fn(g["ka_key"], np.full(4, 255, np.uint8), 0, 255)
        assert np.array_equal(t2b, g["ka_key_t2b"])
        assert np.array_equal(_bits(s), _bits(g["ka_key_scale"])) and np.array_equal(_bits(z), _bits(g["ka_key_zero"]))
    for fn in (O.quantize_value, O.quantize_value_np):
        p, s, z = fn(g["ka_value"])
        assert np.array_equal(p, g["ka_value_packed"])
        assert np.array_equal(_bits(s), _bits(g["ka_value_scale"])) and np.array_equal(_bits(z), _bits(g["ka_value_zero"]))


def test_oracle_reproduces_quant_block():
    g = _load("quant_block.npz")
    dk, sen = int(g["d_boost"]), int(g["sentinel"])
    for fn in (O.quantize_key, O.quantize_key_np):
        t2b, th, s, z = fn(g["key"].T.copy(), g["boost_idx"], dk, sen)
        assert np.array_equal(t2b, g["t2b"]) and np.array_equal(th, g["thigh"])
        assert np.array_equal(_bits(s), _bits(g["key_scale"])) and np.array_equal(_bits(z), _bits(g["key_zero"]))
    pk, sv, zv = O.quantize_value(g["value"])
    assert np.array_equal(pk, g["packed"])
    assert np.array_equal(_bits(sv), _bits(g["value_scale"])) and np.array_equal(_bits(zv), _bits(g["value_zero"]))


@pytest.mark.parametrize("case", ["ref", "prod"])
def test_oracle_reproduces_decode(case):
    g = _load("decode_small.npz")
    c = {k[len(case) + 1:]: v for k, v in g.items() if k.startswith(case + "_")}
    H, Hq, D, G = c["shape"].tolist()
    out = O.paged_attention(c["q"], c["pages"], c["kb"], c["kh"], c["km"], c["vp"], c["vm"], c["bi"],
                            int(c["d_boost"]), c["sk"], c["sv"], c["tk"], c["tv"], Hq, H, D)
    np.testing.assert_allclose(np.asarray(out, np.float32), c["out"], rtol=0, atol=1e-6)


@pytest.mark.gpu
def test_hip_quantize_matches_golden(dev):
    from kitty.kernels import quantize_key_page, quantize_value_page
    from kitty.kernels.ops import pool_store, quantize_into_pools
    g = _load("quant_block.npz")
    dk, sen = int(g["d_boost"]), int(g["sentinel"])
    D = G = 128
    key = torch.from_numpy(g["key"]).to(dev)            # (G, D) token-major
    val = torch.from_numpy(g["value"]).to(dev)
    bi = torch.from_numpy(g["boost_idx"]).to(dev)
    # batch path (token-major blocks, the 128 x 128 kernel)
    kb = torch.zeros(1, 1, D, G // 4, dtype=torch.uint8, device=dev)
    kh = torch.zeros(1, 1, dk, G // 4, dtype=torch.uint8, device=dev)
    km = torch.zeros(1, 1, 2, D, dtype=torch.float16, device=dev)
    vp = torch.zeros(1, 1, G, D // 4, dtype=torch.uint8, device=dev)
    vm = torch.zeros(1, 1, G, 2, dtype=torch.float16, device=dev)
    quantize_into_pools(pool_store(kb, kh, km, vp, vm), key[None, None], val[None, None], bi[None],
                        torch.zeros(1, dtype=torch.int32, device=dev), sen)
    # reference-shaped single-block calls (channel-major key view, the generic kernel)
    t2b = torch.zeros(D, G // 4, dtype=torch.uint8, device=dev)
    th = torch.zeros(dk, G // 4, dtype=torch.uint8, device=dev)
    s, z = torch.zeros(D, dtype=torch.float16, device=dev), torch.zeros(D, dtype=torch.float16, device=dev)
    quantize_key_page(key.t().contiguous(), bi, dk, sen, t2b, th, s, z)
    pk = torch.zeros(G, D // 4, dtype=torch.uint8, device=dev)
    sv, zv = torch.zeros(G, dtype=torch.float16, device=dev), torch.zeros(G, dtype=torch.float16, device=dev)
    quantize_value_page(val, pk, sv, zv)
    torch.cuda.synchronize()
    for got in ((kb[0, 0], kh[0, 0], km[0, 0, 0], km[0, 0, 1]), (t2b, th, s, z)):
        assert np.array_equal(got[0].cpu().numpy(), g["t2b"]) and np.array_equal(got[1].cpu().numpy(), g["thigh"])
        assert np.array_equal(_bits(got[2].cpu().numpy()), _bits(g["key_scale"]))
        assert np.array_equal(_bits(got[3].cpu().numpy()), _bits(g["key_zero"]))
    for got in ((vp[0, 0], vm[0, 0, :, 0], vm[0, 0, :, 1]), (pk, sv, zv)):
        assert np.array_equal(got[0].cpu().numpy(), g["packed"])
        assert np.array_equal(_bits(got[1].cpu().numpy()), _bits(g["value_scale"]))
        assert np.array_equal(_bits(got[2].cpu().numpy()), _bits(g["value_zero"]))


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["ref", "prod"])
def test_hip_decode_matches_golden(dev, case):
    from kitty.kernels import paged_attention
    g = _load("decode_small.npz")
    c = {k[len(case) + 1:]: v for k, v in g.items() if k.startswith(case + "_")}
    H, Hq, D, G = c["shape"].tolist()
    t = {k: torch.from_numpy(c[k]).to(dev) for k in ("q", "kb", "kh", "km", "vp", "vm", "bi", "sk", "sv", "tk", "tv")}
    out = paged_attention(t["q"], c["pages"].tolist(), t["kb"], t["kh"], t["km"], t["vp"], t["vm"], t["bi"],
                          int(c["d_boost"]), t["sk"], t["sv"], t["tk"], t["tv"], Hq, H, D)
    got = out.float().cpu().numpy()
    ref = c["out"]
    assert np.isfinite(got).all()
    assert (np.abs(got - ref) <= 2e-3 + 1e-2 * np.abs(ref)).all(), np.abs(got - ref).max()
