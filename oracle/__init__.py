"""CPU oracle for the blockwise-FP8 W8A8 path -- TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``liboracle.so`` (a C restatement of the reference's CPU
golden code, see oracle.c) and, when it has been built, over
``_ref/libinferop_ref.so`` (the reference's own reference.cpp compiled from its
sources by oracle/Makefile).  Only tests/, ``__graft_entry__.smoke()`` and
bench.py's ``cpu_baseline`` leg import this package, as the checker or as the
timed CPU baseline; the product (``inferop_amd``) never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libinferop_ref.so")

_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_u64 = ctypes.c_uint64

_lib = None
_ref = None


def build() -> None:
    """Compile liboracle.so (and the reference build when its sources exist)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _ptr(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_e4m3_to_float.restype = ctypes.c_float
        L.orc_e4m3_to_float.argtypes = [ctypes.c_uint8]
        L.orc_float_to_e4m3.restype = ctypes.c_uint8
        L.orc_float_to_e4m3.argtypes = [ctypes.c_float]
        L.orc_grid_encode.restype = ctypes.c_uint8
        L.orc_grid_encode.argtypes = [ctypes.c_float]
        L.orc_bf16_to_float.restype = ctypes.c_float
        L.orc_bf16_to_float.argtypes = [ctypes.c_uint16]
        L.orc_float_to_bf16.restype = ctypes.c_uint16
        L.orc_float_to_bf16.argtypes = [ctypes.c_float]
        L.orc_half_to_float.restype = ctypes.c_float
        L.orc_half_to_float.argtypes = [ctypes.c_uint16]
        L.orc_float_to_half.restype = ctypes.c_uint16
        L.orc_float_to_half.argtypes = [ctypes.c_float]
        L.orc_quant_fp8_per_token_group.argtypes = [_u8p, _f32p, _f32p, _i64, _i64, _i32]
        L.orc_dequant_fp8_per_token_group.argtypes = [_f32p, _u8p, _f32p, _i64, _i64, _i32]
        L.orc_w8a8_block_fp8_gemm.argtypes = [_f32p, _u8p, _f32p, _u8p, _f32p, _i64, _i64, _i64,
                                              _i32, _i32, _i32]
        L.orc_w8a8_block_fp8_gemm_rows.argtypes = [_f32p, _u8p, _f32p, _u8p, _f32p, _i64, _i64,
                                                   _i64, _i32, _i32, _i64p, _i64, _i32]
        L.orc_weight_block_quant.argtypes = [_u8p, _f32p, _f32p, _i64, _i64, _i32, _i32]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, ctypes.c_float]
        L.orc_fused_add_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64,
                                            ctypes.c_float]
        L.orc_silu_and_mul.argtypes = [_f32p, _f32p, _i64, _i64]
        L.orc_topk_softmax.argtypes = [ctypes.POINTER(ctypes.c_int32), _f32p, _f32p, _i64, _i32,
                                       _i32, _i32]
        L.orc_sweep_encode_vs_grid.restype = _u64
        L.orc_sweep_encode_vs_grid.argtypes = [_u64, _u64]
        L.orc_encode_checksum.restype = _u64
        L.orc_encode_checksum.argtypes = [_u64, _u64]
        L.orc_encode_range.argtypes = [_u64, _u64, _u8p]
        L.orc_bf16_range.argtypes = [_u64, _u64, _u16p]
        L.orc_half_range.argtypes = [_u64, _u64, _u16p]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    """The compiled reference (only where oracle/Makefile could build it)."""
    global _ref
    if _ref is None:
        R = ctypes.CDLL(REF_PATH)
        R.ref_float_to_e4m3.restype = ctypes.c_uint8
        R.ref_float_to_e4m3.argtypes = [ctypes.c_float]
        R.ref_e4m3_to_float.restype = ctypes.c_float
        R.ref_e4m3_to_float.argtypes = [ctypes.c_uint8]
        R.ref_encode_range.argtypes = [_u64, _u64, _u8p]
        R.ref_bf16_range.argtypes = [_u64, _u64, _u16p]
        R.ref_half_range.argtypes = [_u64, _u64, _u16p]
        R.ref_half_to_float.restype = ctypes.c_float
        R.ref_half_to_float.argtypes = [ctypes.c_uint16]
        R.ref_quant.argtypes = [_u8p, _f32p, _f32p, _i64, _i64, ctypes.c_int]
        R.ref_dequant.argtypes = [_f32p, _u8p, _f32p, _i64, _i64, ctypes.c_int]
        R.ref_gemm.argtypes = [_f32p, _u8p, _f32p, _u8p, _f32p, _i64, _i64, _i64, ctypes.c_int,
                               ctypes.c_int]
        R.ref_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, ctypes.c_float]
        R.ref_fused_add_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64,
                                            ctypes.c_float]
        R.ref_silu_and_mul.argtypes = [_f32p, _f32p, _i64, _i64]
        R.ref_topk_softmax.argtypes = [ctypes.POINTER(ctypes.c_int32), _f32p, _f32p, _i64,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int]
        _ref = R
    return _ref


# ---- numpy-level helpers ----------------------------------------------------

def quant(x: np.ndarray, group_size: int = 128):
    """reference.cpp:65-80 on an fp32 [rows, cols] array -> (q uint8, scales fp32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows, cols // group_size), np.float32)
    lib().orc_quant_fp8_per_token_group(_ptr(q, _u8p), _ptr(s, _f32p), _ptr(x, _f32p), rows, cols,
                                        group_size)
    return q, s


def dequant(q: np.ndarray, s: np.ndarray, group_size: int = 128) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    rows, cols = q.shape
    x = np.empty((rows, cols), np.float32)
    lib().orc_dequant_fp8_per_token_group(_ptr(x, _f32p), _ptr(q, _u8p), _ptr(s, _f32p), rows,
                                          cols, group_size)
    return x


def gemm(a_q, a_s, b_q, b_s, threads: int = 0) -> np.ndarray:
    """reference.cpp:93-110 -> fp32 C [M, N] (fp64 accumulation)."""
    a_q = np.ascontiguousarray(a_q, dtype=np.uint8)
    b_q = np.ascontiguousarray(b_q, dtype=np.uint8)
    a_s = np.ascontiguousarray(a_s, dtype=np.float32)
    b_s = np.ascontiguousarray(b_s, dtype=np.float32)
    m, k = a_q.shape
    n = b_q.shape[0]
    c = np.empty((m, n), np.float32)
    lib().orc_w8a8_block_fp8_gemm(_ptr(c, _f32p), _ptr(a_q, _u8p), _ptr(a_s, _f32p),
                                  _ptr(b_q, _u8p), _ptr(b_s, _f32p), m, n, k, 128, 128, threads)
    return c


def gemm_rows(a_q, a_s, b_q, b_s, rows, threads: int = 0) -> np.ndarray:
    """The oracle GEMM for selected output rows only -> fp32 [len(rows), N]."""
    a_q = np.ascontiguousarray(a_q, dtype=np.uint8)
    b_q = np.ascontiguousarray(b_q, dtype=np.uint8)
    a_s = np.ascontiguousarray(a_s, dtype=np.float32)
    b_s = np.ascontiguousarray(b_s, dtype=np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    m, k = a_q.shape
    n = b_q.shape[0]
    c = np.empty((len(rows), n), np.float32)
    lib().orc_w8a8_block_fp8_gemm_rows(_ptr(c, _f32p), _ptr(a_q, _u8p), _ptr(a_s, _f32p),
                                       _ptr(b_q, _u8p), _ptr(b_s, _f32p), m, n, k, 128, 128,
                                       _ptr(rows, _i64p), len(rows), threads)
    return c


def weight_block_quant(w: np.ndarray):
    """tests/test_gemm.cpp:28-45 -> (b_q uint8 [N, K], b_s fp32 [ceil(N/128), K/128])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    bq = np.empty((n, k), np.uint8)
    bs = np.empty(((n + 127) // 128, k // 128), np.float32)
    lib().orc_weight_block_quant(_ptr(bq, _u8p), _ptr(bs, _f32p), _ptr(w, _f32p), n, k, 128, 128)
    return bq, bs


def e4m3_decode_table() -> np.ndarray:
    L = lib()
    return np.array([L.orc_e4m3_to_float(b) for b in range(256)], np.float32)


def ref_quant(x: np.ndarray, group_size: int = 128):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows, cols // group_size), np.float32)
    ref().ref_quant(_ptr(q, _u8p), _ptr(s, _f32p), _ptr(x, _f32p), rows, cols, group_size)
    return q, s


def ref_dequant(q: np.ndarray, s: np.ndarray, group_size: int = 128) -> np.ndarray:
    """The reference's own dequantizer (reference.cpp:82-91, compiled into
    oracle/_ref) on q [rows, cols] uint8 and s [rows, cols/gs] fp32."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    rows, cols = q.shape
    x = np.empty((rows, cols), np.float32)
    ref().ref_dequant(_ptr(x, _f32p), _ptr(q, _u8p), _ptr(s, _f32p), rows, cols, group_size)
    return x


def ref_gemm(a_q, a_s, b_q, b_s) -> np.ndarray:
    a_q = np.ascontiguousarray(a_q, dtype=np.uint8)
    b_q = np.ascontiguousarray(b_q, dtype=np.uint8)
    a_s = np.ascontiguousarray(a_s, dtype=np.float32)
    b_s = np.ascontiguousarray(b_s, dtype=np.float32)
    m, k = a_q.shape
    n = b_q.shape[0]
    c = np.empty((m, n), np.float32)
    ref().ref_gemm(_ptr(c, _f32p), _ptr(a_q, _u8p), _ptr(a_s, _f32p), _ptr(b_q, _u8p),
                   _ptr(b_s, _f32p), m, n, k, 128, 128)
    return c


def silu_and_mul(gate_up: np.ndarray) -> np.ndarray:
    """reference.cpp:55-64 on fp32 [tokens, 2d] -> [tokens, d]."""
    gu = np.ascontiguousarray(gate_up, dtype=np.float32)
    t, d2 = gu.shape
    out = np.empty((t, d2 // 2), np.float32)
    lib().orc_silu_and_mul(_ptr(out, _f32p), _ptr(gu, _f32p), t, d2 // 2)
    return out


def fused_add_rmsnorm(residual: np.ndarray, x: np.ndarray, weight: np.ndarray,
                      eps: float = 1e-6):
    """reference.cpp:23-35 -> (new residual, out), inputs untouched."""
    res = np.array(residual, dtype=np.float32, order="C", copy=True)
    xr = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    rows, cols = res.shape
    out = np.empty_like(res)
    lib().orc_fused_add_rmsnorm(_ptr(res, _f32p), _ptr(out, _f32p), _ptr(xr, _f32p),
                                _ptr(w, _f32p), rows, cols, eps)
    return res, out


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """reference.cpp:11-21."""
    xr = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    rows, cols = xr.shape
    out = np.empty_like(xr)
    lib().orc_rmsnorm(_ptr(out, _f32p), _ptr(xr, _f32p), _ptr(w, _f32p), rows, cols, eps)
    return out


def topk_softmax(logits: np.ndarray, topk: int, renormalize: bool = True):
    """reference.cpp:152-181 -> (ids int32 [tokens, topk], weights fp32 [tokens, topk])."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    t, e = lg.shape
    ids = np.empty((t, topk), np.int32)
    w = np.empty((t, topk), np.float32)
    lib().orc_topk_softmax(ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), _ptr(w, _f32p),
                           _ptr(lg, _f32p), t, e, topk, 1 if renormalize else 0)
    return ids, w
