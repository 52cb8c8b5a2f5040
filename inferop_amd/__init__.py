"""inferop_amd: MI355X-native (gfx950) blockwise-FP8 W8A8 path of inferop.

The product is libinferop.so: the drop-in C++ API of include/inferop/ops.h,
its C-ABI twin include/inferop/inferop_c.h, and the HIP kernels behind them.
This package builds it (``inferop_amd.build``) and binds its C-ABI from
Python (``inferop_amd.ops``, same names as the reference's operators).
"""
from ._lib import LIB_PATH, LibraryNotBuilt, lib  # noqa: F401
from .ops import (  # noqa: F401
    dequant_fp8_per_token_group, dequantize, device_count, device_name, device_sm_version,
    diag_mfma_loop, diag_read_stream, diag_stripe_read, dtype, fused_add_rmsnorm_quant_fp8, gemm,
    gemm_config_name, gemm_num_configs, gemm_select, grouped_gemm_masked_select,
    grouped_gemm_select, has_cuda, InferopError, quant_fp8_per_token_group,
    quant_fp8_weight_block, quant_gemm_launches, quant_w8a8_block_fp8_gemm, quantize,
    quantize_weight, silu_and_mul_quant_fp8,
    splitk_workspace_info, Status,
    topk_softmax, w8a8_block_fp8_gemm, w8a8_block_fp8_gemm_config, w8a8_block_fp8_gemm_noalloc,
    w8a8_block_fp8_grouped_gemm, w8a8_block_fp8_grouped_gemm_config,
    w8a8_block_fp8_grouped_gemm_masked, w8a8_block_fp8_grouped_gemm_masked_config)
