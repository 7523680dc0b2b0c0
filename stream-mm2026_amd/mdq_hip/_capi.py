"""ctypes binding of libstquant_hip.so (C ABI declared in include/stquant_hip.h).

torch is imported before the library is loaded so that the HIP runtime torch
already mapped (SONAME libamdhip64.so.7) is the one the library binds to; the
stream handles passed in are torch's.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libstquant_hip.so")

STQ_OK, STQ_ERR_INVALID, STQ_ERR_HIP = 0, 1, 2
NOALLOC_MAX_TENSORS = 4096        # STQ_NOALLOC_MAX_TENSORS
ROUND_NEAREST, ROUND_STOCHASTIC = 0, 1

DTYPE_CODES = {
    torch.float32: 0,
    torch.bfloat16: 1,
    torch.float16: 2,
    torch.uint8: 3,
    torch.int8: 4,
    torch.int16: 5,
    torch.uint16: 6,
    torch.int32: 7,
    torch.uint32: 8,
    torch.int64: 9,
}

# Every symbol include/stquant_hip.h declares.
EXPORTED_SYMBOLS = (
    "stq_fused_mdq_adamw",
    "stq_multi_tensor_mdq_adamw",
    "stq_multi_tensor_mdq_adamw_noalloc",
    "stq_multi_tensor_mdq_adamw_restore",
    "stq_multi_tensor_grad_stats",
    "stq_multi_tensor_convert_codes",
    "stq_last_error",
    "stq_abi_version",
    "stq_step_table_uploads",
    "stq_device_math",
    "stq_device_math_digests",
    "stq_device_log_approx_error",
    "stq_device_hw_ulp_error",
    "stq_host_math",
    "stq_host_round_half_away",
    "stq_host_div_code_range",
    "stq_host_philox4x32_10",
)


# STQ_ABI_VERSION of include/stquant_hip.h this package is written against
ABI_VERSION = 4


class StqTensor(ctypes.Structure):
    """Mirror of ``stq_tensor``."""

    _fields_ = [
        ("p", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("exp_avg", ctypes.c_void_p),
        ("exp_avg_sq", ctypes.c_void_p),
        ("scale_m", ctypes.c_void_p),
        ("scale_v", ctypes.c_void_p),
        ("v_min", ctypes.c_void_p),
        ("numel", ctypes.c_int64),
        ("grad_numel", ctypes.c_int64),
        ("exp_avg_numel", ctypes.c_int64),
        ("exp_avg_sq_numel", ctypes.c_int64),
        ("scale_m_numel", ctypes.c_int64),
        ("scale_v_numel", ctypes.c_int64),
        ("v_min_numel", ctypes.c_int64),
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("lr", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("step", ctypes.c_int32),
        ("bits", ctypes.c_int32),
        ("tensor_id", ctypes.c_uint32),
        ("elem_offset", ctypes.c_int64),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built (there is no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"MDQ HIP library not built: {LIB_PATH} is missing "
            "(build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "or `make -C stream-mm2026_amd/csrc`)")
    L = ctypes.CDLL(LIB_PATH)
    vp, i64, i32, u32, u64, f32 = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                    ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float)
    L.stq_fused_mdq_adamw.argtypes = [
        vp, vp, i32, i64, i64,
        vp, i32, i64,
        vp, i32, i64,
        vp, i64, vp, i64, vp, i64,
        f32, f32, f32, f32, f32,
        i32, i32, i32,
        vp, i64,
        i32, u64, u32, vp]
    L.stq_fused_mdq_adamw.restype = ctypes.c_int
    L.stq_multi_tensor_mdq_adamw.argtypes = [
        ctypes.POINTER(StqTensor), i32, i32, i32, i32, i32, i32, u64, vp, i64, vp]
    L.stq_multi_tensor_mdq_adamw.restype = ctypes.c_int
    L.stq_multi_tensor_mdq_adamw_noalloc.argtypes = L.stq_multi_tensor_mdq_adamw.argtypes
    L.stq_multi_tensor_mdq_adamw_noalloc.restype = ctypes.c_int
    L.stq_multi_tensor_mdq_adamw_restore.argtypes = [
        ctypes.POINTER(StqTensor), vp, i32, i32, i32, i32, i32, i32, u64, vp, i64, vp]
    L.stq_multi_tensor_mdq_adamw_restore.restype = ctypes.c_int
    L.stq_multi_tensor_convert_codes.argtypes = [vp, i32, vp]
    L.stq_multi_tensor_convert_codes.restype = ctypes.c_int
    L.stq_multi_tensor_grad_stats.argtypes = [vp, vp, i32, i32, vp, vp]
    L.stq_multi_tensor_grad_stats.restype = ctypes.c_int
    L.stq_last_error.argtypes = []
    L.stq_last_error.restype = ctypes.c_char_p
    L.stq_abi_version.argtypes = []
    L.stq_abi_version.restype = ctypes.c_int
    L.stq_step_table_uploads.argtypes = [vp]
    L.stq_step_table_uploads.restype = ctypes.c_int
    L.stq_device_math.argtypes = [i32, vp, vp, i64, vp]
    L.stq_device_math.restype = ctypes.c_int
    L.stq_device_math_digests.argtypes = [i32, u32, u32, u32, vp, vp]
    L.stq_device_math_digests.restype = ctypes.c_int
    L.stq_device_log_approx_error.argtypes = [u32, u32, ctypes.c_double, vp, vp]
    L.stq_device_log_approx_error.restype = ctypes.c_int
    L.stq_device_hw_ulp_error.argtypes = [i32, u32, u32, vp, vp]
    L.stq_device_hw_ulp_error.restype = ctypes.c_int
    L.stq_host_math.argtypes = [i32, vp, vp, i64]
    L.stq_host_math.restype = None
    L.stq_host_round_half_away.argtypes = [vp, vp, vp, i64, i32]
    L.stq_host_round_half_away.restype = None
    L.stq_host_div_code_range.argtypes = [vp, vp, i64, i32]
    L.stq_host_div_code_range.restype = None
    L.stq_host_philox4x32_10.argtypes = [vp, vp, vp]
    L.stq_host_philox4x32_10.restype = None
    if L.stq_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has ABI version {L.stq_abi_version()}, this package needs "
                           f"{ABI_VERSION}: rebuild it")
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != STQ_OK:
        msg = lib().stq_last_error().decode("utf-8", "replace")
        raise RuntimeError(msg)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dt]
    except KeyError:
        raise RuntimeError(f"MDQ: unsupported dtype {dt}") from None


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
