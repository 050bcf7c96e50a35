"""ctypes binding of libkitty_hip.so (C ABI declared in include/kitty_hip.h).

The library is the only compute path of this package for device tensors:
if it is missing, calls on device tensors raise instead of falling back to
CPU code (CPU tensors are dispatched by the callers to ``kernels.cpu``
before anything here runs).  Error codes map to the exception types the reference raises on the
same conditions (RuntimeError for an exhausted pool, KeyError for a missing
page, ValueError/AssertionError-like ValueError for bad shapes).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# KITTY_HIP_LIBRARY selects another build of the same ABI (e.g. a tuning variant).
LIB_PATH = os.environ.get("KITTY_HIP_LIBRARY") or os.path.join(_HERE, "libkitty_hip.so")

KITTY_ABI_VERSION = 6
KITTY_OK = 0
KITTY_E_INVALID = -1
KITTY_E_HIP = -2
KITTY_E_UNSUPPORTED = -3
KITTY_E_EXHAUSTED = -4
KITTY_E_NOT_FOUND = -5
KITTY_DECODE_UNIQUE_BOOST_ROWS = 1
KITTY_DTYPE_F16 = 0
KITTY_DTYPE_BF16 = 1
KITTY_OUT_F16, KITTY_OUT_F32, KITTY_OUT_BF16 = 0, 1, 2
KITTY_DECODE_PATH_GENERIC, KITTY_DECODE_PATH_MFMA = 0, 1


def dtype_code(t: torch.Tensor, name: str) -> int:
    """KITTY_DTYPE_* of a 16-bit float tensor (fp16 or bf16, the two dtypes
    KittyConfig allows, config.py:76)."""
    if t.dtype == torch.float16:
        return KITTY_DTYPE_F16
    if t.dtype == torch.bfloat16:
        return KITTY_DTYPE_BF16
    raise ValueError(f"{name} must be float16 or bfloat16, got {t.dtype}")

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p


class PageStore(ctypes.Structure):
    """kitty_page_store: where quantised pages are written (strided pools/views)."""
    _fields_ = [
        ("key_low", _vp), ("key_low_s_page", _i64), ("key_low_s_head", _i64), ("key_low_s_row", _i64),
        ("key_high", _vp), ("key_high_s_page", _i64), ("key_high_s_head", _i64), ("key_high_s_row", _i64),
        ("key_scale", _vp), ("key_zero", _vp),
        ("key_meta_s_page", _i64), ("key_meta_s_head", _i64), ("key_meta_s_chan", _i64),
        ("value", _vp), ("value_s_page", _i64), ("value_s_head", _i64), ("value_s_row", _i64),
        ("value_scale", _vp), ("value_zero", _vp),
        ("value_meta_s_page", _i64), ("value_meta_s_head", _i64), ("value_meta_s_tok", _i64),
        ("num_pages", _i64),
        ("num_kv_heads", _i32), ("head_dim", _i32), ("page_tokens", _i32), ("d_boost", _i32),
        ("meta_dtype", _i32),
    ]


class QuantBatch(ctypes.Structure):
    """kitty_quant_batch: the (outer, inner) grid of fp16 blocks of one spill."""
    _fields_ = [
        ("key", _vp), ("key_s_outer", _i64), ("key_s_inner", _i64), ("key_s_tok", _i64), ("key_s_chan", _i64),
        ("value", _vp), ("value_s_outer", _i64), ("value_s_inner", _i64), ("value_s_tok", _i64),
        ("value_s_chan", _i64),
        ("boost_idx", _vp), ("boost_s_outer", _i64), ("boost_s_inner", _i64),
        ("page_ids", _vp), ("n_outer", _i32), ("n_inner", _i32), ("value_rows", _i32), ("sentinel", _i32),
        ("src_dtype", _i32), ("outer_per_seq", _i32), ("key_s_seq", _i64), ("value_s_seq", _i64),
        ("value_page_ids", _vp), ("value_shift", _i32),
    ]


class Fp16Seg(ctypes.Structure):
    _fields_ = [("ptr", _vp), ("s_seq", _i64), ("s_head", _i64), ("s_tok", _i64)]


class DecodeArgs(ctypes.Structure):
    """kitty_decode_args: one batched paged-decode step."""
    _fields_ = [
        ("q", _vp), ("q_s_seq", _i64), ("q_s_head", _i64),
        ("out", _vp), ("out_s_seq", _i64), ("out_s_head", _i64),
        ("key_low", _vp), ("key_high", _vp), ("key_meta", _vp), ("value", _vp), ("value_meta", _vp),
        ("num_pool_pages", _i64),
        ("block_table", _vp), ("bt_stride", _i64), ("num_pages", _vp), ("boost_idx", _vp),
        ("sink_k", Fp16Seg), ("sink_v", Fp16Seg), ("tail_k", Fp16Seg), ("tail_v", Fp16Seg),
        ("sink_len", _vp), ("tail_len", _vp), ("sink_capacity", _i32), ("tail_capacity", _i32),
        ("batch", _i32), ("num_q_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("page_tokens", _i32), ("d_boost", _i32), ("max_pages", _i32), ("pages_per_split", _i32),
        ("flags", _i32), ("sm_scale", ctypes.c_float),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("num_pages_v", _vp), ("tail_len_v", _vp), ("tail_v_capacity", _i32),
        ("meta_dtype", _i32), ("act_dtype", _i32),
    ]


class SlotLayout(ctypes.Structure):
    _fields_ = [("s_slot", _i64), ("s_head", _i64), ("s_tok", _i64)]


class AppendArgs(ctypes.Structure):
    """kitty_append_args: one token for each of B sequences into its FP16 buffers."""
    _fields_ = [
        ("key", _vp), ("value", _vp),
        ("key_s_seq", _i64), ("key_s_head", _i64), ("value_s_seq", _i64), ("value_s_head", _i64),
        ("slots", _vp),
        ("sink_k", _vp), ("sink_v", _vp), ("sink_layout", SlotLayout),
        ("buf_k", _vp), ("buf_v", _vp), ("buf_layout", SlotLayout),
        ("sink_fill", _vp), ("buf_len", _vp), ("overflow", _vp),
        ("batch", _i32), ("num_kv_heads", _i32), ("head_dim", _i32), ("sink_size", _i32), ("buf_tokens", _i32),
        ("num_slots", _i32),
        ("val_len", _vp), ("val_buf", _vp), ("val_layout", SlotLayout), ("val_tokens", _i32),
    ]


EXPORTED_SYMBOLS = (
    "kitty_abi_version", "kitty_last_error", "kitty_quantize_kv_blocks",
    "kitty_dequantize_key_page", "kitty_dequantize_value_page",
    "kitty_decode_workspace_size", "kitty_decode_path", "kitty_paged_decode", "kitty_paged_decode_splits",
    "kitty_paged_decode_merge", "kitty_paged_decode_noalloc", "kitty_append_tokens", "kitty_channel_abs_sum",
    "kitty_channel_abs_sum_workspace_size", "kitty_channel_abs_sum_deferred_size", "kitty_channel_abs_sum_deferred",
    "kitty_channel_abs_sum_flush", "kitty_store_i32",
)

_lib: Optional[ctypes.CDLL] = None


class KittyHipError(RuntimeError):
    """A libkitty_hip call failed inside the HIP runtime."""


def load() -> ctypes.CDLL:
    """Load libkitty_hip.so once; raise ImportError if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(or `make -C kitty-kv_amd/csrc`). Device tensors have no CPU fallback.")
    L = ctypes.CDLL(LIB_PATH)
    L.kitty_abi_version.restype = ctypes.c_int
    L.kitty_last_error.restype = ctypes.c_char_p
    L.kitty_quantize_kv_blocks.argtypes = [ctypes.POINTER(PageStore), ctypes.POINTER(QuantBatch), _vp]
    L.kitty_dequantize_key_page.argtypes = [ctypes.POINTER(PageStore), _i64, _i32, _vp, _vp, _i64, _i32, _vp]
    L.kitty_dequantize_value_page.argtypes = [ctypes.POINTER(PageStore), _i64, _i32, _vp, _i64, _i32, _vp]
    L.kitty_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.POINTER(ctypes.c_size_t)]
    L.kitty_decode_path.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.POINTER(ctypes.c_int32)]
    L.kitty_paged_decode.argtypes = [ctypes.POINTER(DecodeArgs), _vp]
    L.kitty_paged_decode_splits.argtypes = [ctypes.POINTER(DecodeArgs), _vp]
    L.kitty_paged_decode_merge.argtypes = [ctypes.POINTER(DecodeArgs), _vp]
    L.kitty_paged_decode_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), _vp]
    L.kitty_append_tokens.argtypes = [ctypes.POINTER(AppendArgs), _vp]
    L.kitty_channel_abs_sum_workspace_size.argtypes = [_i32, _i32, _i32, _i32, ctypes.POINTER(ctypes.c_size_t)]
    L.kitty_channel_abs_sum.argtypes = [_vp, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _vp, _vp,
                                        ctypes.c_size_t, _vp]
    L.kitty_channel_abs_sum_deferred_size.argtypes = [_i32, _i32, ctypes.POINTER(ctypes.c_size_t)]
    L.kitty_channel_abs_sum_deferred.argtypes = L.kitty_channel_abs_sum.argtypes
    L.kitty_channel_abs_sum_flush.argtypes = [_vp, _i32, _i32, _vp, _vp]
    L.kitty_store_i32.argtypes = [_vp, _vp, _i32, _vp]
    if L.kitty_abi_version() != KITTY_ABI_VERSION:
        raise ImportError(f"libkitty_hip ABI {L.kitty_abi_version()} != {KITTY_ABI_VERSION}")
    _lib = L
    return L


def check(rc: int) -> None:
    """Raise the exception that matches a KITTY_E_* code."""
    if rc == KITTY_OK:
        return
    msg = load().kitty_last_error().decode(errors="replace")
    if rc == KITTY_E_INVALID:
        raise ValueError(msg)
    if rc == KITTY_E_UNSUPPORTED:
        raise NotImplementedError(msg)
    if rc == KITTY_E_EXHAUSTED:
        raise RuntimeError(msg)
    if rc == KITTY_E_NOT_FOUND:
        raise KeyError(msg)
    raise KittyHipError(msg)


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on the same ROCm device: the HIP path never
    falls back to the CPU (CPU inputs are dispatched before this check)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "kitty (MI355X build) computes only on ROCm device tensors; got a tensor on "
                f"{t.device}. Move the pools and inputs to 'cuda'.")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """hipStream_t of the current stream on a ROCm device (torch's raw
    query when it has one: building a torch Stream object costs ~5 µs)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()
