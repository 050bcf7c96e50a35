"""Key page quantisation (reference ``kitty/kernels/quantize_key.py``).

Per-channel min-max over the G tokens of a page, INT4 for boosted channels
(``boost_idx[d] < sentinel``) and INT2 otherwise, packed into the dense-sparse
layout: low 2 bits of every channel -> ``Tensor_2bits`` (D, G/4), high 2 bits
of boosted channels -> row ``boost_idx[d]`` of ``Tensor_High_2bits``
(D_boost, G/4).  Computed by the HIP kernel ``quantize_kv_kernel`` for device
tensors and by ``kernels.cpu`` for CPU tensors; results are bit-identical to
the reference's ``quantize_key_page_torch``.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .. import _hip
from . import cpu
from .ops import _dtype16, _need, quantize_into_pools


def _key_store(D: int, G: int, D_boost: int, out_baseline, out_boost, out_scale, out_zero) -> _hip.PageStore:
    _need(tuple(out_baseline.shape) == (D, G // 4) and out_baseline.dtype == torch.uint8
          and out_baseline.stride(1) == 1, "out_baseline must be uint8 (D, G//4) with contiguous rows")
    _need(tuple(out_boost.shape) == (D_boost, G // 4) and out_boost.dtype == torch.uint8
          and (D_boost == 0 or out_boost.stride(1) == 1), "out_boost must be uint8 (D_boost, G//4)")
    _need(out_scale.shape == (D,) and out_zero.shape == (D,) and out_scale.stride(0) == out_zero.stride(0),
          "out_scale / out_zero must be (D,) views with equal strides")
    meta_dtype = _dtype16("out_scale and out_zero", out_scale, out_zero)
    s = _hip.PageStore()
    s.key_low, s.key_low_s_row = out_baseline.data_ptr(), out_baseline.stride(0)
    s.key_high = out_boost.data_ptr() if D_boost > 0 else 0
    s.key_high_s_row = out_boost.stride(0) if D_boost > 0 else 0
    s.key_scale, s.key_zero, s.key_meta_s_chan = out_scale.data_ptr(), out_zero.data_ptr(), out_scale.stride(0)
    s.num_pages = 1
    s.num_kv_heads, s.head_dim, s.page_tokens, s.d_boost = 1, D, G, D_boost
    s.meta_dtype = meta_dtype
    return s


def quantize_key_page(key: torch.Tensor, boost_idx: torch.Tensor, D_boost: int, sentinel: int,
                      out_baseline: torch.Tensor, out_boost: torch.Tensor,
                      out_scale: torch.Tensor, out_zero: torch.Tensor) -> None:
    """Quantise one (D, G) fp16 or bf16 key block into pre-allocated outputs
    (reference quantize_key.py:217-269); float16 or bfloat16 out_scale /
    out_zero receive the fp16 scale and zero point converted to their dtype,
    as the reference's copy_ does.  A CPU key is quantised by the torch code
    of ``kernels.cpu`` and copied into the outputs wherever they live
    (quantize_key.py:263-269)."""
    D, G = key.shape
    assert G % 4 == 0, "G must be divisible by 4 for uint8 packing"
    if key.device.type == "cpu":
        res = cpu.quantize_key_blocks(key, boost_idx.cpu(), D_boost, sentinel)
        for out, r in zip((out_baseline, out_boost, out_scale, out_zero), res):
            out.copy_(r)
        return
    dev = _hip.require_device(key, boost_idx, out_baseline, out_boost, out_scale, out_zero)
    store = _key_store(D, G, D_boost, out_baseline, out_boost, out_scale, out_zero)
    page0 = torch.zeros(1, dtype=torch.int32, device=dev)
    quantize_into_pools(store, key.t()[None, None], None, boost_idx.reshape(1, D), page0, sentinel)


def quantize_key_page_torch(key: torch.Tensor, boost_idx: torch.Tensor, D_boost: int,
                            sentinel: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Same signature and outputs as the reference's pure-PyTorch quantiser
    (quantize_key.py:38-124), computed by the HIP kernel on the key's device
    (by ``kernels.cpu`` for a CPU key)."""
    if key.device.type == "cpu":
        return cpu.quantize_key_blocks(key, boost_idx.cpu(), D_boost, sentinel)
    _hip.require_device(key, boost_idx)
    D, G = key.shape
    dev = key.device
    t2b = torch.empty(D, G // 4, dtype=torch.uint8, device=dev)
    thigh = torch.empty(D_boost, G // 4, dtype=torch.uint8, device=dev)
    scale = torch.empty(D, dtype=torch.float16, device=dev)
    zero = torch.empty(D, dtype=torch.float16, device=dev)
    quantize_key_page(key, boost_idx, D_boost, sentinel, t2b, thigh, scale, zero)
    return t2b, thigh, scale, zero
