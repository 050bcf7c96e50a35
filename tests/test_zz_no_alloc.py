"""kitty_paged_decode_noalloc (decode with the library's own device scratch
instead of a caller workspace) against kitty_paged_decode on the same
arguments, through the C ABI: bit-exact, since both run the same kernels
and work plan.  Calls follow one another on one stream, each with a
different (smaller) batch, so a stale partial left in the shared scratch
by an earlier call would show up."""
import ctypes

import numpy as np
import pytest
import torch

from test_decode_gpu import _batched_case

pytestmark = pytest.mark.gpu


def _plan(dev, c, **kw):
    from kitty.kernels.ops import DecodePlan
    kb, kh, km, vp, vm = [t.to(dev) for t in c["pools"]]
    B = c["q"].shape[0]
    return DecodePlan(c["q"].to(dev), c["bt"].to(dev), torch.tensor(c["n_pages"], dtype=torch.int32, device=dev),
                      kb, kh, km, vp, vm, c["bi"].to(dev), c["sk"].to(dev), c["sv"].to(dev),
                      torch.full((B,), c["S"], dtype=torch.int32, device=dev), c["tk"].to(dev), c["tv"].to(dev),
                      torch.tensor(c["tails"], dtype=torch.int32, device=dev), **kw)


def _noalloc(plan):
    from kitty import _hip
    out = torch.full_like(plan.out, float("nan"))
    a = _hip.DecodeArgs.from_buffer_copy(plan.args)
    a.out = out.data_ptr()
    a.workspace, a.workspace_bytes = None, 0      # ignored by the no-alloc entry point
    _hip.check(_hip.load().kitty_paged_decode_noalloc(ctypes.byref(a), _hip.stream_ptr(plan.device)))
    return out


@pytest.mark.parametrize("kernel", ["mfma", "generic"])
def test_noalloc_matches_workspace_decode(dev, kernel):
    from kitty.kernels.ops import DecodePlan  # noqa: F401  (library loads first)
    kw = {}
    if kernel == "generic":
        shapes = [(5, 8, 4, 64, 32, 8, [40 + 9 * 32 + 3, 40 + 2 * 32, 40, 40 + 17 * 32 + 31, 40 + 5 * 32 + 1]),
                  (2, 8, 4, 64, 32, 8, [40 + 3 * 32 + 7, 40 + 32])]
    else:
        # the last two: groups of 20 query heads per KV head, which run as
        # sub-groups of 16 and 4, each a split + merge through the one scratch
        shapes = [(16, 32, 8, 128, 128, 16, [32 + 40 * 128 + 100] * 12 + [32, 32 + 128, 32 + 7 * 128 + 5, 33]),
                  (3, 32, 8, 128, 128, 16, [32 + 5 * 128 + 3, 32 + 2 * 128, 32 + 11 * 128 + 127]),
                  (2, 40, 2, 128, 128, 16, [32 + 9 * 128 + 40, 32 + 3 * 128 + 5]),
                  (1, 40, 2, 128, 128, 16, [32 + 2 * 128 + 7])]
    for i, (B, Hq, H, D, G, dk, ctx) in enumerate(shapes):
        print(f"noalloc {kernel} call {i}: B={B} Hq={Hq} H={H} D={D}", flush=True)
        c = _batched_case(dev, 70 + i, B, Hq, H, D, G, dk, ctx, S=32 if D == 128 else 40)
        plan = _plan(dev, c, **kw)
        ref = plan.run().clone()
        got = _noalloc(plan)
        torch.cuda.synchronize()
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(got, ref), f"{kernel} call {i}: max |diff| {(got.float() - ref.float()).abs().max()}"


def test_noalloc_rejects_oversize_batch(dev):
    """A batch whose workspace exceeds the scratch fails with KITTY_E_INVALID
    before any launch; the next call still works."""
    from kitty import _hip
    c = _batched_case(dev, 80, 2, 8, 2, 128, 128, 16, [32 + 3 * 128 + 5, 32 + 128])
    plan = _plan(dev, c)
    a = _hip.DecodeArgs.from_buffer_copy(plan.args)
    a.batch = 20000                              # workspace far above 64 MiB (not launched)
    assert _hip.load().kitty_paged_decode_noalloc(ctypes.byref(a), _hip.stream_ptr(plan.device)) == \
        _hip.KITTY_E_INVALID
    assert b"maximum" in _hip.load().kitty_last_error()
    ref = plan.run().clone()
    got = _noalloc(plan)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
