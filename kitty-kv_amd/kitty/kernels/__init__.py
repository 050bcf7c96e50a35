"""Kernel entry points with the reference's names (kitty/kernels/__init__.py:10-29).

All of them run HIP kernels from libkitty_hip.so on ROCm device tensors and
the vectorised torch code of ``kernels.cpu`` on CPU tensors, as the
reference dispatches by device.  The ``*_torch`` names keep the reference's
return-value signatures (they allocate their outputs) and compute where
their inputs live.
"""
from .quantize_key import quantize_key_page, quantize_key_page_torch
from .dequantize_key import dequantize_key_page, dequantize_key_page_torch
from .quantize_value import quantize_value_page, quantize_value_page_torch, dequantize_value_page_torch
from .attention import paged_attention, paged_attention_reference, paged_attention_batched

__all__ = [
    "quantize_key_page",
    "quantize_key_page_torch",
    "dequantize_key_page",
    "dequantize_key_page_torch",
    "quantize_value_page",
    "quantize_value_page_torch",
    "dequantize_value_page_torch",
    "paged_attention",
    "paged_attention_reference",
    "paged_attention_batched",
]
