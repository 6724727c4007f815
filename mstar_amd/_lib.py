"""ctypes binding of ``libmstar_moe.so`` (the C-ABI in include/mstar_moe.h).

The library is built in-tree by :mod:`mstar_amd.build`.  There is no
fallback: if the library is missing or a call fails, an exception is raised.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmstar_moe.so")

# dtype codes (MSTAR_DTYPE_*)
DT_F32, DT_BF16, DT_F16, DT_I32, DT_I64, DT_FP8, DT_FP8_AS_BF16 = 0, 1, 2, 3, 4, 5, 6
QUANT_NONE, QUANT_FP8_W8A8, QUANT_W4A16 = 0, 1, 2

_TORCH_DT = {
    torch.float32: DT_F32,
    torch.bfloat16: DT_BF16,
    torch.float16: DT_F16,
    torch.int32: DT_I32,
    torch.int64: DT_I64,
    torch.float8_e4m3fn: DT_FP8,
}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_vp = ctypes.c_void_p
_f32 = ctypes.c_float

# (name, argtypes) for every exported entry point; kept in the order of the
# header so a test can compare the two.
SIGNATURES = {
    "mstar_moe_last_error": (ctypes.c_char_p, []),
    "mstar_moe_abi_version": (_c_int, []),
    "mstar_moe_topk_softmax": (_c_int, [_vp, _c_int, _c_i64, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp]),
    "mstar_moe_router": (
        _c_int, [_vp, _c_int, _c_i64, _c_i64, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp]),
    "mstar_moe_topk_softmax_quant": (
        _c_int, [_vp, _c_int, _c_i64, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp,
                 _vp]),
    "mstar_moe_align_block_size": (
        _c_int, [_vp, _c_int, _c_i64, _c_int, _c_int, _vp, _c_i64, _vp, _c_i64, _vp, _vp, _vp, _vp,
                 ctypes.c_size_t, _vp]),
    "mstar_moe_align_scratch_size": (_c_int, [_c_i64, _c_int, ctypes.POINTER(ctypes.c_size_t)]),
    "mstar_moe_route": (
        _c_int, [_vp, _c_int, _c_i64, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _vp, _c_i64,
                 _vp, _c_i64, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "mstar_moe_route_scratch_size": (_c_int, [_c_i64, _c_int, _c_int, ctypes.POINTER(ctypes.c_size_t)]),
    "mstar_moe_act_and_mul": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_i64, _c_int, _vp]),
    "mstar_moe_sum_reduce": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_i64, _c_i64, _f32, _vp]),
    "mstar_moe_grouped_gemm": (
        _c_int, [_vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64,
                 _c_int, _c_int, _c_int, _c_int, _vp]),
    "mstar_moe_gemm": (
        _c_int, [_vp, _c_int, _vp, _vp, _c_int, _vp, _vp, _c_int, _vp, _c_int, _vp, _vp, _vp, _vp,
                 _vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
                 _c_int, _vp]),
    "mstar_moe_stream_gemm": (
        _c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_i64, _c_int, _c_i64,
                 _c_i64, _c_int, _c_int, _c_int, _vp]),
    "mstar_moe_stream_layer": (
        _c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_i64, _c_int,
                 _c_int, _vp, _vp, _vp, _vp]),
    "mstar_moe_layer_sync_words": (_c_int, [_c_int, ctypes.POINTER(_c_i64)]),
    "mstar_moe_layer_wait_failures": (_c_int, [ctypes.POINTER(_c_int)]),
    "mstar_moe_debug_layer_test_mode": (_c_int, [_c_int]),
    "mstar_fused_moe_workspace_size": (
        _c_int, [_c_i64, _c_i64, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_int,
                 ctypes.POINTER(ctypes.c_size_t)]),
    "mstar_fused_moe": (
        _c_int, [_vp, _c_int, _c_i64, _c_i64, _vp, _vp, _c_int, _c_i64, _c_int, _vp, _vp, _vp,
                 _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, ctypes.c_size_t, _vp]),
    "mstar_moe_layer_workspace_size": (
        _c_int, [_c_i64, _c_i64, _c_int, _c_i64, _c_int, _c_int, _c_int,
                 ctypes.POINTER(ctypes.c_size_t)]),
    "mstar_moe_layer": (
        _c_int, [_vp, _c_int, _c_i64, _c_i64, _vp, _c_int, _c_int, _vp, _vp, _c_int, _c_i64, _c_int,
                 _vp, _vp, _c_int, _c_int, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "mstar_moe_block": (
        _c_int, [_vp, _c_int, _c_i64, _c_i64, _vp, _c_int, _vp, _vp, _c_int, _c_i64, _c_int,
                 _vp, _vp, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "mstar_moe_layer_noalloc": (
        _c_int, [_vp, _c_int, _c_i64, _c_i64, _vp, _c_int, _c_int, _vp, _vp, _c_int, _c_i64, _c_int,
                 _vp, _vp, _c_int, _c_int, _vp, _vp, _vp, _vp]),
    "mstar_quant_fp8_per_token_group": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_int, _vp, _vp, _vp]),
    "mstar_quant_fp8_per_token": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _vp, _vp, _vp]),
    "mstar_fp8_scaled_mm": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
}

_lib = None
_lock = threading.Lock()


class MstarError(RuntimeError):
    """A libmstar_moe call returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Load the shared library (once) and declare every signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"libmstar_moe.so not found at {LIB_PATH}; build it with "
                    "`python -m mstar_amd.build` (hipcc, gfx950)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _TORCH_DT[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def stream_of(t: torch.Tensor) -> int:
    """The calling thread's current HIP stream on ``t``'s device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().mstar_moe_last_error().decode(errors="replace")
        if status == 1:
            raise ValueError(f"{what}: {msg}")
        raise MstarError(f"{what} failed (status {status}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("mstar_amd kernels run on the GPU; got a CPU tensor")
