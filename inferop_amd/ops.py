"""Python mirror of the reference's ``inferop`` operator API for the FP8 path.

Same names, argument order and meaning as include/inferop/ops.h (reference
ops.h:19-25, 64-70, 81-84): tensors are device pointers (ints) or torch
tensors, ``dt`` / ``out_dt`` are ``dtype`` values, ``stream`` defaults to the
current torch stream.  Like the reference, the raw calls never raise on a bad
shape or dtype: they do nothing and return the C-ABI status code
(``Status.OK`` when the kernels were launched).  ``quantize``, ``dequantize``
and ``gemm`` are tensor-level conveniences that allocate outputs with torch
and raise on any error.

Every call goes to the HIP kernels in libinferop.so; there is no CPU path.
"""
from __future__ import annotations

import ctypes
import enum

from ._lib import lib


class dtype(enum.IntEnum):
    fp32 = 0
    fp16 = 1
    bf16 = 2
    fp8_e4m3 = 3


class Status(enum.IntEnum):
    OK = 0
    ERR_SHAPE = 1
    ERR_DTYPE = 2
    ERR_DEVICE = 3
    ERR_LAUNCH = 4
    ERR_ARGUMENT = 5


class InferopError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        msg = lib().inferop_status_string(int(status)).decode()
        super().__init__(f"{what}: {msg} (status {int(status)})")


def _ptr(t) -> int:
    if t is None:
        return 0
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int:
    if stream is None:
        try:
            import torch
            if torch.cuda.is_available():
                return torch.cuda.current_stream().cuda_stream
        except Exception:  # torch without a device: null stream
            pass
        return 0
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


# ---- ops.h:19-25 ------------------------------------------------------------
def has_cuda() -> bool:
    return bool(lib().inferop_has_device())


def device_count() -> int:
    return lib().inferop_device_count()


def device_name(ordinal: int = 0) -> str:
    return lib().inferop_device_name(ordinal).decode()


def device_sm_version(ordinal: int = 0) -> int:
    return lib().inferop_device_arch(ordinal)


# ---- ops.h:64-65 ------------------------------------------------------------
def quant_fp8_per_token_group(q, scales, x, dt, rows: int, cols: int, group_size: int = 128,
                              stream=None) -> int:
    return lib().inferop_quant_fp8_per_token_group(
        _ptr(q), _ptr(scales), _ptr(x), int(dt), rows, cols, group_size, _stream(stream))


# ---- ops.h:68-70 ------------------------------------------------------------
def dequant_fp8_per_token_group(x, dt, q, scales, rows: int, cols: int, group_size: int = 128,
                                stream=None) -> int:
    return lib().inferop_dequant_fp8_per_token_group(
        _ptr(x), int(dt), _ptr(q), _ptr(scales), rows, cols, group_size, _stream(stream))


# ---- ops.h:81-84 ------------------------------------------------------------
def w8a8_block_fp8_gemm(c, a_q, a_scales, b_q, b_scales, m: int, n: int, k: int,
                        group_size: int = 128, block_n: int = 128, out_dt=dtype.bf16,
                        stream=None) -> int:
    return lib().inferop_w8a8_block_fp8_gemm(
        _ptr(c), _ptr(a_q), _ptr(a_scales), _ptr(b_q), _ptr(b_scales), m, n, k, group_size,
        block_n, int(out_dt), _stream(stream))


def quant_w8a8_block_fp8_gemm(c, q, scales, x, dt, b_q, b_scales, m: int, n: int, k: int,
                              group_size: int = 128, block_n: int = 128, out_dt=dtype.bf16,
                              stream=None) -> int:
    """quant_fp8_per_token_group then w8a8_block_fp8_gemm in one call (no
    reference counterpart): the same q / scales / c, one launch up to 8 rows."""
    return lib().inferop_quant_w8a8_block_fp8_gemm(
        _ptr(c), _ptr(q), _ptr(scales), _ptr(x), int(dt), _ptr(b_q), _ptr(b_scales), m, n, k,
        group_size, block_n, int(out_dt), _stream(stream))


def quant_gemm_launches(m: int, n: int, k: int) -> int:
    """Kernel launches quant_w8a8_block_fp8_gemm makes for this shape (1 or 2)."""
    return lib().inferop_quant_w8a8_block_fp8_gemm_launches(m, n, k)


# ---- allocation-free GEMM (no reference counterpart) -----------------------------
def w8a8_block_fp8_gemm_noalloc(c, a_q, a_scales, b_q, b_scales, m: int, n: int, k: int,
                                group_size: int = 128, block_n: int = 128, out_dt=dtype.bf16,
                                stream=None) -> int:
    """w8a8_block_fp8_gemm without any device allocation (split-K scratch in
    a fixed per-GPU array; no reference counterpart, for callers that cannot
    allocate).  Split-K calls that overlap in time on one GPU race."""
    return lib().inferop_w8a8_block_fp8_gemm_noalloc(
        _ptr(c), _ptr(a_q), _ptr(a_scales), _ptr(b_q), _ptr(b_scales), m, n, k, group_size,
        block_n, int(out_dt), _stream(stream))


# ---- MoE routing (reference ops.h:102-110) ---------------------------------------
def topk_softmax(topk_ids, topk_weights, logits, tokens: int, num_experts: int, topk: int,
                 renormalize: bool = True, stream=None) -> int:
    return lib().inferop_topk_softmax(_ptr(topk_ids), _ptr(topk_weights), _ptr(logits), tokens,
                                      num_experts, topk, 1 if renormalize else 0, _stream(stream))


# ---- extension: weight block quantizer (the reference's test recipe,
# tests/test_gemm.cpp:28-45; no counterpart in its ops.h) ---------------------------
def quant_fp8_weight_block(b_q, b_scales, w, dt, n: int, k: int, group_size: int = 128,
                           block_n: int = 128, stream=None) -> int:
    return lib().inferop_quant_fp8_weight_block(
        _ptr(b_q), _ptr(b_scales), _ptr(w), int(dt), n, k, group_size, block_n, _stream(stream))


# ---- extension: grouped GEMM over MoE experts, contiguous layout (the
# reference's roadmap item, docs/ROADMAP.md:39; no counterpart in its ops.h) ----
def w8a8_block_fp8_grouped_gemm(c, a_q, a_scales, b_q, b_scales, expert_offsets, m: int, n: int,
                                k: int, num_experts: int, group_size: int = 128,
                                block_n: int = 128, out_dt=dtype.bf16, stream=None) -> int:
    return lib().inferop_w8a8_block_fp8_grouped_gemm(
        _ptr(c), _ptr(a_q), _ptr(a_scales), _ptr(b_q), _ptr(b_scales), _ptr(expert_offsets), m, n,
        k, num_experts, group_size, block_n, int(out_dt), _stream(stream))


def w8a8_block_fp8_grouped_gemm_masked(c, a_q, a_scales, b_q, b_scales, masked_m, max_m: int,
                                       n: int, k: int, num_experts: int, expected_m: int = 0,
                                       group_size: int = 128, block_n: int = 128,
                                       out_dt=dtype.bf16, stream=None) -> int:
    return lib().inferop_w8a8_block_fp8_grouped_gemm_masked(
        _ptr(c), _ptr(a_q), _ptr(a_scales), _ptr(b_q), _ptr(b_scales), _ptr(masked_m), max_m, n,
        k, num_experts, expected_m, group_size, block_n, int(out_dt), _stream(stream))


# ---- extension: producers fused with the quantizer (the reference runs
# silu_and_mul / fused_add_rmsnorm, ops.h:33-55, then quant_fp8_per_token_group) ----
def silu_and_mul_quant_fp8(q, scales, gate_up, dt, tokens: int, d: int, group_size: int = 128,
                           stream=None) -> int:
    return lib().inferop_silu_and_mul_quant_fp8(_ptr(q), _ptr(scales), _ptr(gate_up), int(dt),
                                                tokens, d, group_size, _stream(stream))


def fused_add_rmsnorm_quant_fp8(residual, q, scales, x, weight, dt, rows: int, cols: int,
                                eps: float = 1e-6, group_size: int = 128, stream=None) -> int:
    return lib().inferop_fused_add_rmsnorm_quant_fp8(
        _ptr(residual), _ptr(q), _ptr(scales), _ptr(x), _ptr(weight), int(dt), rows, cols,
        eps, group_size, _stream(stream))


# ---- tuning entry points (no reference counterpart) ------------------------------
def gemm_num_configs() -> int:
    return lib().inferop_gemm_num_configs()


def gemm_config_name(config: int) -> str:
    return lib().inferop_gemm_config_name(config).decode()


def gemm_select(m: int, n: int, k: int):
    cfg, split = ctypes.c_int32(), ctypes.c_int32()
    st = lib().inferop_gemm_select(m, n, k, ctypes.byref(cfg), ctypes.byref(split))
    if st != Status.OK:
        raise InferopError(st, "gemm_select")
    return cfg.value, split.value


def splitk_workspace_info():
    """(slots_used, slots_total, slot_bytes) of the current device's split-K
    workspace pool."""
    used, total, nbytes = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    st = lib().inferop_splitk_workspace_info(ctypes.byref(used), ctypes.byref(total),
                                             ctypes.byref(nbytes))
    if st != Status.OK:
        raise InferopError(st, "splitk_workspace_info")
    return used.value, total.value, nbytes.value


def w8a8_block_fp8_gemm_config(c, a_q, a_scales, b_q, b_scales, m: int, n: int, k: int,
                               out_dt, config: int, split_k: int = 1, stream=None) -> int:
    return lib().inferop_w8a8_block_fp8_gemm_config(
        _ptr(c), _ptr(a_q), _ptr(a_scales), _ptr(b_q), _ptr(b_scales), m, n, k, int(out_dt),
        config, split_k, _stream(stream))


def w8a8_block_fp8_grouped_gemm_config(c, a_q, a_scales, b_q, b_scales, expert_offsets, m: int,
                                       n: int, k: int, num_experts: int, out_dt, config: int,
                                       stream=None) -> int:
    return lib().inferop_w8a8_block_fp8_grouped_gemm_config(
        _ptr(c), _ptr(a_q), _ptr(a_scales), _ptr(b_q), _ptr(b_scales), _ptr(expert_offsets), m, n,
        k, num_experts, int(out_dt), config, _stream(stream))


def w8a8_block_fp8_grouped_gemm_masked_config(c, a_q, a_scales, b_q, b_scales, masked_m,
                                              max_m: int, n: int, k: int, num_experts: int,
                                              out_dt, config: int, stream=None) -> int:
    return lib().inferop_w8a8_block_fp8_grouped_gemm_masked_config(
        _ptr(c), _ptr(a_q), _ptr(a_scales), _ptr(b_q), _ptr(b_scales), _ptr(masked_m), max_m, n,
        k, num_experts, int(out_dt), config, _stream(stream))


def grouped_gemm_select(m: int, n: int, k: int, num_experts: int) -> int:
    cfg = ctypes.c_int32()
    st = lib().inferop_grouped_gemm_select(m, n, k, num_experts, ctypes.byref(cfg))
    if st != Status.OK:
        raise InferopError(st, "grouped_gemm_select")
    return cfg.value


def grouped_gemm_masked_select(max_m: int, n: int, k: int, num_experts: int,
                               expected_m: int = 0) -> int:
    cfg = ctypes.c_int32()
    st = lib().inferop_grouped_gemm_masked_select(max_m, n, k, num_experts, expected_m,
                                                  ctypes.byref(cfg))
    if st != Status.OK:
        raise InferopError(st, "grouped_gemm_masked_select")
    return cfg.value


def selftest_fp8_codec(counts, lo: int = 0, hi: int = 1 << 32, stream=None) -> int:
    return lib().inferop_selftest_fp8_codec(lo, hi, _ptr(counts), _stream(stream))


def diag_read_stream(src, nbytes: int, blocks: int, sink, stream=None) -> int:
    """One plain read of nbytes of src (the HBM read ceiling of a stream)."""
    return lib().inferop_diag_read_stream(_ptr(src), nbytes, blocks, _ptr(sink), _stream(stream))


def diag_stripe_read(b, n: int, k: int, pattern: int, stripes: int, sink, stream=None) -> int:
    """One read of the [n, k] bytes of b, one 8-wave workgroup per 16-row
    stripe, all loads in flight, in access pattern 0-3; stripes > 0 keeps the
    data L2-resident (a compute unit's load rate)."""
    return lib().inferop_diag_stripe_read(_ptr(b), n, k, pattern, stripes, _ptr(sink),
                                          _stream(stream))


def diag_mfma_loop(iters: int, blocks: int, promote: bool, sink, stream=None) -> int:
    """The GEMM's MFMA inner loop from registers (the matrix-core ceiling)."""
    return lib().inferop_diag_mfma_loop(iters, blocks, 1 if promote else 0, _ptr(sink),
                                        _stream(stream))


# ---- tensor-level conveniences ---------------------------------------------------
def _torch_dtype_code(t) -> dtype:
    import torch
    return {torch.float32: dtype.fp32, torch.float16: dtype.fp16,
            torch.bfloat16: dtype.bf16}[t]


def quantize(x, group_size: int = 128, stream=None):
    """x: [rows, cols] fp32/fp16/bf16 device tensor -> (q uint8, scales fp32)."""
    import torch
    rows, cols = x.shape
    x = x.contiguous()
    q = torch.empty((rows, cols), dtype=torch.uint8, device=x.device)
    s = torch.empty((rows, cols // group_size), dtype=torch.float32, device=x.device)
    st = quant_fp8_per_token_group(q, s, x, _torch_dtype_code(x.dtype), rows, cols, group_size,
                                   stream)
    if st != Status.OK:
        raise InferopError(st, "quant_fp8_per_token_group")
    return q, s


def quantize_weight(w, stream=None):
    """w: [n, k] fp32/fp16/bf16 device tensor -> (b_q uint8 [n, k], b_scales fp32
    [ceil(n/128), k/128]), the weight format the GEMM consumes."""
    import torch
    n, k = w.shape
    w = w.contiguous()
    q = torch.empty((n, k), dtype=torch.uint8, device=w.device)
    s = torch.empty(((n + 127) // 128, k // 128), dtype=torch.float32, device=w.device)
    st = quant_fp8_weight_block(q, s, w, _torch_dtype_code(w.dtype), n, k, 128, 128, stream)
    if st != Status.OK:
        raise InferopError(st, "quant_fp8_weight_block")
    return q, s


def dequantize(q, scales, out_dtype=None, group_size: int = 128, stream=None):
    import torch
    out_dtype = out_dtype or torch.bfloat16
    rows, cols = q.shape
    x = torch.empty((rows, cols), dtype=out_dtype, device=q.device)
    st = dequant_fp8_per_token_group(x, _torch_dtype_code(out_dtype), q, scales, rows, cols,
                                     group_size, stream)
    if st != Status.OK:
        raise InferopError(st, "dequant_fp8_per_token_group")
    return x


def gemm(a_q, a_s, b_q, b_s, out_dtype=None, stream=None):
    """C[M,N] = blockwise-FP8 product of a_q [M,K] and b_q [N,K]."""
    import torch
    out_dtype = out_dtype or torch.bfloat16
    m, k = a_q.shape
    n = b_q.shape[0]
    c = torch.empty((m, n), dtype=out_dtype, device=a_q.device)
    st = w8a8_block_fp8_gemm(c, a_q, a_s, b_q, b_s, m, n, k, 128, 128,
                             _torch_dtype_code(out_dtype), stream)
    if st != Status.OK:
        raise InferopError(st, "w8a8_block_fp8_gemm")
    return c
