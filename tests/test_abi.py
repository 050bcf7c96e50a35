"""CPU checks of the C ABI: the library loads, exports every function that
include/kitty_hip.h declares, and rejects bad arguments before touching a GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    text = open(os.path.join(ROOT, "include", "kitty_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kitty_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = _declared_functions()
    for n in ("kitty_abi_version", "kitty_last_error", "kitty_quantize_kv_blocks", "kitty_paged_decode",
              "kitty_decode_workspace_size", "kitty_dequantize_key_page", "kitty_dequantize_value_page"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from kitty import _hip
    L = _hip.load()
    for name in _declared_functions():
        assert hasattr(L, name), name
    assert set(_hip.EXPORTED_SYMBOLS) <= set(_declared_functions())
    assert L.kitty_abi_version() == _hip.KITTY_ABI_VERSION


def test_invalid_arguments_are_rejected_without_launch():
    from kitty import _hip
    L = _hip.load()
    assert L.kitty_quantize_kv_blocks(None, None, None) == _hip.KITTY_E_INVALID
    assert b"NULL" in L.kitty_last_error()
    st = _hip.PageStore()
    st.head_dim, st.page_tokens, st.num_kv_heads = 130, 128, 1
    b = _hip.QuantBatch()
    assert L.kitty_quantize_kv_blocks(ctypes.byref(st), ctypes.byref(b), None) == _hip.KITTY_E_INVALID
    st.head_dim = 128
    b.n_outer, b.n_inner, b.page_ids, b.outer_per_seq = 1, 1, 16, -1   # the id pointer is never read here
    assert L.kitty_quantize_kv_blocks(ctypes.byref(st), ctypes.byref(b), None) == _hip.KITTY_E_INVALID
    assert b"outer_per_seq" in L.kitty_last_error()
    b.outer_per_seq, b.value_shift = 0, 129
    assert L.kitty_quantize_kv_blocks(ctypes.byref(st), ctypes.byref(b), None) == _hip.KITTY_E_INVALID
    assert b"value_shift" in L.kitty_last_error()
    b.value_shift = 64                                                  # no value blocks to shift
    assert L.kitty_quantize_kv_blocks(ctypes.byref(st), ctypes.byref(b), None) == _hip.KITTY_E_INVALID
    assert b"value_shift needs" in L.kitty_last_error()
    a = _hip.DecodeArgs()
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.page_tokens = 1, 6, 4, 128, 128
    assert L.kitty_paged_decode(ctypes.byref(a), None) == _hip.KITTY_E_INVALID
    a.num_q_heads, a.head_dim = 8, 512
    assert L.kitty_paged_decode(ctypes.byref(a), None) == _hip.KITTY_E_UNSUPPORTED
    # spill bookkeeping: bad lists fail before any launch; empty lists are no-ops
    import numpy as np
    addrs = np.array([0x1000, 0x1002], np.int64)       # never dereferenced: the second is misaligned
    vals = np.array([1, 2], np.int32)
    assert L.kitty_store_i32(addrs.ctypes.data, vals.ctypes.data, 2, None) == _hip.KITTY_E_INVALID
    assert b"misaligned" in L.kitty_last_error()
    assert L.kitty_store_i32(None, None, -1, None) == _hip.KITTY_E_INVALID
    assert L.kitty_store_i32(None, None, 0, None) == _hip.KITTY_OK
    with pytest.raises(NotImplementedError):
        _hip.check(_hip.KITTY_E_UNSUPPORTED)
    with pytest.raises(RuntimeError):
        _hip.check(_hip.KITTY_E_EXHAUSTED)
    with pytest.raises(KeyError):
        _hip.check(_hip.KITTY_E_NOT_FOUND)


def test_workspace_size_formula():
    from kitty.kernels.ops import decode_workspace_bytes
    row = (128 + 2) * 4  # O + (m, l) per partial row, fp32
    # Config 3 shape on 256 CUs.  Uniform plan (generic kernel): 15 splits of
    # 17 pages + 1 FP16 split per (b, q head).  Unit-balanced plan (MFMA
    # kernel, 8 waves per CU): GQ rows per partial t < 2 (2048 resident waves
    # + 128 pairs), plus the (first, last) partial table of the pairs.  The
    # size covers both.
    uniform = 16 * 32 * 16 * row
    balanced = 2 * (2048 + 128) * 4 * row + 128 * 2 * 4
    assert decode_workspace_bytes(16, 32, 8, 128, 128, 16, 255) == max(uniform, balanced)
    # pages_per_split = 200: uniform splits capped at 64 pages (4 + 1 per
    # head); balanced: at least 200 units per wave, 128 pairs x ceil(256 / 200)
    # waves
    uniform = 16 * 32 * (4 + 1) * row
    balanced = 2 * (128 * 2 + 128) * 4 * row + 128 * 2 * 4
    assert decode_workspace_bytes(16, 32, 8, 128, 128, 16, 255, pages_per_split=200) == max(uniform, balanced)
    # pages_per_split = 4: 128 pairs x ceil(units / 4) waves, where a pair's
    # units are its pages, its FP16 units (8 per 128 sink + tail tokens of
    # capacity) and one: the FP16 capacities enter the size
    balanced0 = 2 * (128 * 64 + 128) * 4 * row + 128 * 2 * 4              # (255 + 0 + 1) / 4
    balanced1 = 2 * (128 * 67 + 128) * 4 * row + 128 * 2 * 4              # (255 + 10 + 1) / 4
    assert decode_workspace_bytes(16, 32, 8, 128, 128, 16, 255, pages_per_split=4) == balanced0
    assert decode_workspace_bytes(16, 32, 8, 128, 128, 16, 255, pages_per_split=4, sink_capacity=32,
                                  tail_capacity=128) == balanced1
    # an independent value stream plans with the value tail's capacity (32 + 256 tokens: 18 FP16 units)
    balanced2 = 2 * (128 * 69 + 128) * 4 * row + 128 * 2 * 4              # ceil((255 + 18 + 1) / 4)
    assert decode_workspace_bytes(16, 32, 8, 128, 128, 16, 255, pages_per_split=4, sink_capacity=32,
                                  tail_capacity=128, tail_v_capacity=256) == balanced2
    # a shape only the generic kernel takes (GQA 2): uniform plan alone
    assert decode_workspace_bytes(16, 16, 8, 128, 128, 16, 255) == 16 * 16 * 16 * row


def test_hip_boundary_rejects_cpu_tensors():
    """The HIP path never computes on the CPU: its device check refuses CPU
    tensors (the public functions dispatch CPU tensors to kernels.cpu before
    it), and a DecodePlan built directly over CPU tensors raises."""
    import torch
    from kitty import _hip
    from kitty.kernels.ops import DecodePlan
    with pytest.raises(RuntimeError, match="ROCm device"):
        _hip.require_device(torch.zeros(4, dtype=torch.float16))
    z8 = torch.zeros(1, 1, 16, 2, dtype=torch.uint8)
    i1 = torch.zeros(1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="ROCm device"):
        DecodePlan(torch.zeros(1, 1, 16).half(), torch.zeros(1, 1, dtype=torch.int32), i1, z8, z8[:, :, :0],
                   torch.zeros(1, 1, 2, 16).half(), torch.zeros(1, 1, 8, 4, dtype=torch.uint8),
                   torch.zeros(1, 1, 8, 2).half(), torch.zeros(1, 16, dtype=torch.uint8),
                   *(torch.zeros(1, 1, 0, 16).half(),) * 2, i1, *(torch.zeros(1, 1, 0, 16).half(),) * 2, i1)


def test_cpu_dispatch_never_loads_the_hip_library():
    """CPU tensors run kitty.kernels.cpu without the HIP library, while any
    device call needs it: with the library path pointing nowhere, CPU calls
    work and loading the library raises ImportError (no fallback)."""
    import subprocess
    import sys
    code = (
        "import sys, torch; sys.path.insert(0, %r)\n"
        "from kitty import _hip\n"
        "from kitty.kernels import quantize_value_page_torch, paged_attention\n"
        "p, s, z = quantize_value_page_torch(torch.full((8, 16), 3.0).half())\n"
        "assert (p == 0xFF).all()\n"
        "z8 = torch.zeros(1, 1, 16, 2, dtype=torch.uint8)\n"
        "out = paged_attention(torch.zeros(1, 16).half(), [], z8, z8[:, :, :0], torch.zeros(1, 1, 2, 16).half(),"
        " torch.zeros(1, 1, 8, 4, dtype=torch.uint8), torch.zeros(1, 1, 8, 2).half(),"
        " torch.zeros(1, 16, dtype=torch.uint8), 0, torch.ones(1, 2, 16).half(), torch.ones(1, 2, 16).half(),"
        " torch.zeros(1, 0, 16).half(), torch.zeros(1, 0, 16).half(), 1, 1, 16)\n"
        "assert (out == 1).all()\n"
        "assert _hip._lib is None\n"
        "try:\n    _hip.load()\nexcept ImportError as e:\n    print('no-lib', 'no CPU fallback' in str(e))\n"
    ) % os.path.join(ROOT, "kitty-kv_amd")
    env = dict(os.environ, KITTY_HIP_LIBRARY=os.path.join(ROOT, "no_such_library.so"))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "no-lib True"


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with a message (status 2)
    before touching a device."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_noalloc_rejects_batches_beyond_its_scratch():
    """kitty_paged_decode_noalloc refuses, before touching a device, a batch
    whose workspace exceeds its fixed scratch."""
    from kitty import _hip
    L = _hip.load()
    a = _hip.DecodeArgs()
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.page_tokens, a.d_boost = 20000, 32, 8, 128, 128, 16
    a.max_pages, a.bt_stride = 255, 255
    a.block_table = a.key_low = a.key_high = a.key_meta = a.value = a.value_meta = 1  # never dereferenced
    assert L.kitty_paged_decode_noalloc(ctypes.byref(a), None) == _hip.KITTY_E_INVALID
    assert b"maximum is 67108864" in L.kitty_last_error()


def test_groups_above_16_run_only_through_the_whole_decode():
    """A group of 40 query heads per KV head runs as sub-groups of 16, 16 and
    8 through kitty_paged_decode; the split-only and merge-only entry points
    refuse it before any launch, and the workspace covers the largest
    sub-group's plan."""
    from kitty import _hip
    L = _hip.load()
    a = _hip.DecodeArgs()
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.page_tokens, a.d_boost = 2, 40, 1, 128, 128, 16
    a.max_pages, a.bt_stride = 8, 8
    a.block_table = a.key_low = a.key_high = a.key_meta = a.value = a.value_meta = 16   # never dereferenced
    need40 = ctypes.c_size_t(0)
    _hip.check(L.kitty_decode_workspace_size(ctypes.byref(a), ctypes.byref(need40)))
    a.num_q_heads = 16
    need16 = ctypes.c_size_t(0)
    _hip.check(L.kitty_decode_workspace_size(ctypes.byref(a), ctypes.byref(need16)))
    assert need40.value == need16.value > 0
    a.num_q_heads = 40
    a.q = a.out = a.num_pages = a.boost_idx = a.sink_len = a.tail_len = 16
    a.workspace, a.workspace_bytes = 256, need40.value
    for fn in (L.kitty_paged_decode_splits, L.kitty_paged_decode_merge):
        assert fn(ctypes.byref(a), None) == _hip.KITTY_E_UNSUPPORTED
        assert b"groups above 16" in L.kitty_last_error()
