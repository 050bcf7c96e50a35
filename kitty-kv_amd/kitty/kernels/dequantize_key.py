"""Key page dequantisation (reference ``kitty/kernels/dequantize_key.py``):
k = ((low | high << 2) - z) * s, high bits read from row boost_idx[d] of
Tensor_High_2bits when boost_idx[d] < D_boost.  HIP kernel
``dequantize_key_kernel`` for device tensors, ``kernels.cpu`` for CPU
tensors."""
from __future__ import annotations

import ctypes

import torch

from .. import _hip
from . import cpu
from .ops import _need
from .quantize_key import _key_store


def dequantize_key_page(tensor_2bits: torch.Tensor, tensor_high_2bits: torch.Tensor, scale: torch.Tensor,
                        zero_point: torch.Tensor, boost_idx: torch.Tensor, D_boost: int,
                        out: torch.Tensor) -> None:
    """Dequantise one key page into ``out`` (D, G) of float16, bfloat16 or
    float32 (dequantize_key.py:169-228: the fp32 result converted to out's
    dtype).  A CPU page is dequantised by ``kernels.cpu`` and copied into out
    wherever it lives."""
    D, G4 = tensor_2bits.shape
    if tensor_2bits.device.type == "cpu":
        _need(out.shape == (D, G4 * 4), "out must be (D, G)")
        out.copy_(cpu.dequantize_key_blocks(tensor_2bits, tensor_high_2bits, scale, zero_point, boost_idx.cpu(),
                                            D_boost))
        return
    dev = _hip.require_device(tensor_2bits, tensor_high_2bits, scale, zero_point, boost_idx, out)
    kinds = {torch.float16: _hip.KITTY_OUT_F16, torch.float32: _hip.KITTY_OUT_F32,
             torch.bfloat16: _hip.KITTY_OUT_BF16}
    _need(out.shape == (D, G4 * 4) and out.stride(1) == 1 and out.dtype in kinds,
          "out must be (D, G) float16/bfloat16/float32 with contiguous rows")
    _need(boost_idx.dtype == torch.uint8 and boost_idx.shape == (D,) and boost_idx.is_contiguous(),
          "boost_idx must be contiguous uint8 (D,)")
    store = _key_store(D, G4 * 4, D_boost, tensor_2bits, tensor_high_2bits, scale, zero_point)
    _hip.check(_hip.load().kitty_dequantize_key_page(
        ctypes.byref(store), 0, 0, boost_idx.data_ptr(), out.data_ptr(), out.stride(0),
        kinds[out.dtype], _hip.stream_ptr(dev)))


def dequantize_key_page_torch(tensor_2bits: torch.Tensor, tensor_high_2bits: torch.Tensor, scale: torch.Tensor,
                              zero_point: torch.Tensor, boost_idx: torch.Tensor, D_boost: int) -> torch.Tensor:
    """(D, G) float32, same signature as dequantize_key.py:35-97, on the
    page's device (by ``kernels.cpu`` on the CPU)."""
    if tensor_2bits.device.type == "cpu":
        return cpu.dequantize_key_blocks(tensor_2bits, tensor_high_2bits, scale, zero_point, boost_idx, D_boost)
    D, G4 = tensor_2bits.shape
    out = torch.empty(D, G4 * 4, dtype=torch.float32, device=tensor_2bits.device)
    dequantize_key_page(tensor_2bits, tensor_high_2bits, scale, zero_point, boost_idx, D_boost, out)
    return out
