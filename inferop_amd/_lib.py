"""ctypes binding of libinferop.so's C-ABI (include/inferop/inferop_c.h).

The library is built in-tree by ``python -m inferop_amd.build`` (or
``__graft_entry__.build()``).  There is no fallback: if the shared library is
missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libinferop.so")

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64

# (name, restype, argtypes) for every function declared in inferop_c.h
C_API = [
    ("inferop_status_string", ctypes.c_char_p, [ctypes.c_int]),
    ("inferop_has_device", ctypes.c_int, []),
    ("inferop_device_count", ctypes.c_int, []),
    ("inferop_device_name", ctypes.c_char_p, [ctypes.c_int]),
    ("inferop_device_arch", ctypes.c_int, [ctypes.c_int]),
    ("inferop_quant_fp8_per_token_group", ctypes.c_int,
     [_vp, _vp, _vp, _i32, _i64, _i64, _i32, _vp]),
    ("inferop_dequant_fp8_per_token_group", ctypes.c_int,
     [_vp, _i32, _vp, _vp, _i64, _i64, _i32, _vp]),
    ("inferop_w8a8_block_fp8_gemm", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp]),
    ("inferop_w8a8_block_fp8_gemm_noalloc", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp]),
    ("inferop_quant_w8a8_block_fp8_gemm", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp]),
    ("inferop_quant_w8a8_block_fp8_gemm_launches", ctypes.c_int, [_i64, _i64, _i64]),
    ("inferop_topk_softmax", ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    ("inferop_quant_fp8_weight_block", ctypes.c_int,
     [_vp, _vp, _vp, _i32, _i64, _i64, _i32, _i32, _vp]),
    ("inferop_silu_and_mul_quant_fp8", ctypes.c_int, [_vp, _vp, _vp, _i32, _i64, _i64, _i32, _vp]),
    ("inferop_fused_add_rmsnorm_quant_fp8", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, ctypes.c_float, _i32, _vp]),
    ("inferop_w8a8_block_fp8_grouped_gemm", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _vp]),
    ("inferop_w8a8_block_fp8_grouped_gemm_masked", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _vp]),
    ("inferop_gemm_num_configs", ctypes.c_int, []),
    ("inferop_gemm_config_name", ctypes.c_char_p, [ctypes.c_int]),
    ("inferop_w8a8_block_fp8_gemm_config", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp]),
    ("inferop_w8a8_block_fp8_grouped_gemm_config", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, _vp]),
    ("inferop_grouped_gemm_select", ctypes.c_int, [_i64, _i64, _i64, _i64, _vp]),
    ("inferop_grouped_gemm_masked_select", ctypes.c_int, [_i64, _i64, _i64, _i64, _i64, _vp]),
    ("inferop_w8a8_block_fp8_grouped_gemm_masked_config", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, _vp]),
    ("inferop_gemm_select", ctypes.c_int,
     [_i64, _i64, _i64, ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    ("inferop_splitk_workspace_info", ctypes.c_int,
     [ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_i64)]),
    ("inferop_selftest_fp8_codec", ctypes.c_int, [_u64, _u64, _vp, _vp]),
    ("inferop_diag_read_stream", ctypes.c_int, [_vp, _i64, _i32, _vp, _vp]),
    ("inferop_diag_mfma_loop", ctypes.c_int, [_i32, _i32, _i32, _vp, _vp]),
    ("inferop_diag_stripe_read", ctypes.c_int, [_vp, _i64, _i64, _i32, _i32, _vp, _vp]),
]

_lib = None


class LibraryNotBuilt(RuntimeError):
    pass


def lib():
    """Load libinferop.so (raises LibraryNotBuilt when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryNotBuilt(
                f"{LIB_PATH} is missing: build it with `python -m inferop_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, res, args in C_API:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib
