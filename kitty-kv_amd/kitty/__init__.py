"""Kitty 2-bit KV cache, MI355X (gfx950) implementation of the quantized-KV hot path.

Public names follow the reference package (kitty/__init__.py:7-27).  On ROCm
device tensors all compute runs in libkitty_hip.so (hand-written HIP kernels
for gfx950), with no fallback; CPU tensors (the reference's CPU path,
``KittyConfig.device = "cpu"``) run vectorised torch code
(``kitty.kernels.cpu``).
"""
from .config import KittyConfig
from .layout import Page, PageCentricKVLayoutManager
from .pipeline import KittyInferencePipeline
from .attention import KittyPagedAttention, KittyAttentionFactory
from .sensitivity import KittySensitivityProfiler

__version__ = "0.1.0"
__description__ = (
    "2-bit KV Cache Quantization with per-channel boosted precision and Dense-Sparse memory "
    "decomposition; MI355X HIP kernels.")

__all__ = [
    "KittyConfig",
    "Page",
    "PageCentricKVLayoutManager",
    "KittyInferencePipeline",
    "KittyPagedAttention",
    "KittyAttentionFactory",
    "KittySensitivityProfiler",
]
