"""Value page quantisation (reference ``kitty/kernels/quantize_value.py``).

Per-token INT2 min-max over D channels, 4 channels per byte along D, with a
per-token fp16 (scale, zero point).  Computed by the HIP kernel
``quantize_kv_kernel`` for device tensors and by ``kernels.cpu`` for CPU
tensors; bit-identical to ``quantize_value_page_torch``.
"""
from __future__ import annotations

import ctypes
from typing import Tuple

import torch

from .. import _hip
from . import cpu
from .ops import _dtype16, _need, quantize_into_pools


def _value_store(G: int, D: int, out_packed, out_scale, out_zero) -> _hip.PageStore:
    _need(tuple(out_packed.shape) == (G, D // 4) and out_packed.dtype == torch.uint8
          and out_packed.stride(1) == 1, "out_packed must be uint8 (G, D//4) with contiguous rows")
    _need(out_scale.shape == (G,) and out_zero.shape == (G,) and out_scale.stride(0) == out_zero.stride(0),
          "out_scale / out_zero must be (G,) views with equal strides")
    meta_dtype = _dtype16("out_scale and out_zero", out_scale, out_zero)
    s = _hip.PageStore()
    s.value, s.value_s_row = out_packed.data_ptr(), out_packed.stride(0)
    s.value_scale, s.value_zero, s.value_meta_s_tok = out_scale.data_ptr(), out_zero.data_ptr(), out_scale.stride(0)
    s.num_pages = 1
    s.num_kv_heads, s.head_dim, s.page_tokens, s.d_boost = 1, D, G, 0
    s.meta_dtype = meta_dtype
    return s


def quantize_value_page(value: torch.Tensor, out_packed: torch.Tensor, out_scale: torch.Tensor,
                        out_zero: torch.Tensor) -> None:
    """Quantise one (G, D) fp16 or bf16 value block into pre-allocated
    outputs; the scale / zero views (float16 or bfloat16) may be strided
    (quantize_value.py:197-227).  A CPU value block is quantised by
    ``kernels.cpu`` and copied into the outputs wherever they live."""
    G, D = value.shape
    assert D % 4 == 0, "head_dim D must be divisible by 4 for packing"
    if value.device.type == "cpu":
        for out, r in zip((out_packed, out_scale, out_zero), cpu.quantize_value_blocks(value)):
            out.copy_(r)
        return
    dev = _hip.require_device(value, out_packed, out_scale, out_zero)
    store = _value_store(G, D, out_packed, out_scale, out_zero)
    page0 = torch.zeros(1, dtype=torch.int32, device=dev)
    quantize_into_pools(store, None, value[None, None], None, page0, 0)


def quantize_value_page_torch(value: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Same signature and outputs as quantize_value.py:38-90, computed on the
    value's device (by ``kernels.cpu`` for a CPU block)."""
    if value.device.type == "cpu":
        return cpu.quantize_value_blocks(value)
    _hip.require_device(value)
    G, D = value.shape
    dev = value.device
    packed = torch.empty(G, D // 4, dtype=torch.uint8, device=dev)
    scale = torch.empty(G, dtype=torch.float16, device=dev)
    zero = torch.empty(G, dtype=torch.float16, device=dev)
    quantize_value_page(value, packed, scale, zero)
    return packed, scale, zero


def dequantize_value_page_torch(packed: torch.Tensor, scale: torch.Tensor, zero_point: torch.Tensor) -> torch.Tensor:
    """(G, D) float32 values, (code - z_t) * s_t (quantize_value.py:97-133),
    on the device of the packed page (by ``kernels.cpu`` on the CPU)."""
    if packed.device.type == "cpu":
        return cpu.dequantize_value_blocks(packed, scale, zero_point)
    dev = _hip.require_device(packed, scale, zero_point)
    G, D4 = packed.shape
    out = torch.empty(G, D4 * 4, dtype=torch.float32, device=dev)
    store = _value_store(G, D4 * 4, packed, scale, zero_point)
    _hip.check(_hip.load().kitty_dequantize_value_page(ctypes.byref(store), 0, 0, out.data_ptr(), out.stride(0),
                                                      _hip.KITTY_OUT_F32, _hip.stream_ptr(dev)))
    return out
