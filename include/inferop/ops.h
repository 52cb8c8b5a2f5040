// inferop (MI355X build) : public host API for the blockwise-FP8 W8A8 path.
//
// Drop-in for the reference header include/inferop/ops.h.  Every reference
// function below has the reference's exact C++ signature and default arguments, so the
// Itanium-mangled symbols exported by libinferop.so are the ones a program
// built against the reference links to.  Only the FP8 path is provided
// (quantizer, dequantizer, blockwise GEMM, and the MoE routing that selects
// the experts whose FP8 weights a token multiplies) plus device
// introspection, and
// three extensions: the weight block quantizer the reference keeps in its
// tests, and the two producers of the quantizer's input fused with it.
//
// All tensors are caller-owned device pointers.  `stream` is an opaque
// hipStream_t; nullptr is the null stream.  Calls are asynchronous on that
// stream, never allocate caller-visible memory and never throw.  Errors follow
// the reference: invalid quantizer shapes or dtypes are silent no-ops; invalid
// GEMM shapes print one line to stderr and return; an unsupported GEMM output
// dtype is a silent no-op.  The C-ABI in inferop/inferop_c.h exposes the same
// calls with a status code.
#pragma once

#include "inferop/common.h"

namespace inferop {

// --- device introspection (reference ops.h:19-25) ---------------------------
// True if at least one HIP device is visible and the kernels are built in.
bool has_cuda();
// Number of visible HIP devices (0 when none).
int device_count();
// Marketing name of a device, "-" for an invalid ordinal.
const char* device_name(int ordinal = 0);
// GPU architecture number of a device, parsed from its gcnArchName
// ("gfx950" -> 950); -1 for an invalid ordinal.  The reference returns the
// CUDA SM version here (major*10+minor); callers use it only to compare.
int device_sm_version(int ordinal = 0);

// --- per-token-group FP8 quantization (reference ops.h:57-65) ---------------
//   x:      [rows, cols] in dt (fp32 / fp16 / bf16)
//   q:      [rows, cols] uint8 (E4M3)
//   scales: [rows, cols / group_size] fp32
//   absmax = max |x| over the group (NaN ignored)
//   scale  = absmax == 0 ? 1 : absmax * fl32(1/448)
//   q      = e4m3_rn_sat(x / scale)   (IEEE division)
void quant_fp8_per_token_group(void* q, void* scales, const void* x, dtype dt, int64_t rows,
                               int64_t cols, int group_size = 128, void* stream = nullptr);

// Inverse: x = dt(e4m3_to_float(q) * scale)  (reference ops.h:67-70).
void dequant_fp8_per_token_group(void* x, dtype dt, const void* q, const void* scales,
                                 int64_t rows, int64_t cols, int group_size = 128,
                                 void* stream = nullptr);

// --- W8A8 blockwise-FP8 GEMM (reference ops.h:72-84) ------------------------
//   C[m,n] = sum_k A_q[m,k] * sa[m, k/128] * B_q[n,k] * sb[n/128, k/128]
//   A_q: [M,K] E4M3, sa: [M, K/128] fp32          (per-token-group scales)
//   B_q: [N,K] E4M3, sb: [ceil(N/128), K/128] fp32 (per 128x128 weight block)
//   C:   [M,N] in out_dt (fp32 / fp16 / bf16)
// Requires group_size == block_n == 128 and K % 128 == 0; any M, N > 0.
void w8a8_block_fp8_gemm(void* c, const void* a_q, const void* a_scales, const void* b_q,
                         const void* b_scales, int64_t m, int64_t n, int64_t k,
                         int group_size = 128, int block_n = 128, dtype out_dt = dtype::bf16,
                         void* stream = nullptr);

// --- MoE routing (reference ops.h:102-110) ------------------------------------
//   logits: [tokens, num_experts] fp32, num_experts <= 1024
//   topk_ids: int32 [tokens, topk]; topk_weights: fp32 [tokens, topk]
//   softmax over the experts, the topk most probable (lower index first on
//   ties), weights = probability, divided by their sum when renormalize.
// Invalid sizes (tokens, num_experts <= 0, num_experts > 1024, topk <= 0,
// topk > num_experts) are silent no-ops.
void topk_softmax(int32_t* topk_ids, void* topk_weights, const void* logits, int tokens,
                  int num_experts, int topk, bool renormalize = true, void* stream = nullptr);

// --- extension: 128x128 weight block quantization ----------------------------
// No counterpart in the reference ops.h: the reference quantizes weights in
// its GEMM tests (tests/test_gemm.cpp:28-45); this is that recipe on the GPU,
// producing exactly the B_q / sb the GEMM above consumes.
//   w:        [n, k] in dt (fp32 / fp16 / bf16), 16-byte aligned
//   b_q:      [n, k] uint8 (E4M3), 8-byte aligned
//   b_scales: [ceil(n/128), k/128] fp32
//   absmax = max |w| over the block (NaN ignored)
//   scale  = absmax == 0 ? 1 : absmax * fl32(1/448)
//   b_q    = e4m3_rn_sat(w * fl32(1 / scale))   (product with the reciprocal)
// Requires group_size == block_n == 128 and k % 128 == 0; other shapes,
// dtypes and misaligned pointers are silent no-ops.
void quant_fp8_weight_block(void* b_q, void* b_scales, const void* w, dtype dt, int64_t n,
                            int64_t k, int group_size = 128, int block_n = 128,
                            void* stream = nullptr);

// --- extension: producers fused with the per-token-group quantizer -----------
// No counterparts in the reference ops.h, which runs these as separate calls:
// silu_and_mul (ops.h:51-55) or fused_add_rmsnorm (ops.h:33-37) writing dt,
// then quant_fp8_per_token_group on that output.  The fused calls produce the
// same q / scales as that sequence would from the dt values it stores, without
// the dt tensor in HBM.  group_size must be 128 and d / cols multiples of 128;
// dt tensors 16-byte aligned, q 8-byte aligned; other calls are no-ops.
//
//   gate_up: [tokens, 2d] dt -> q [tokens, d] E4M3, scales [tokens, d/128]
//   out = silu(gate_up[:, :d]) * gate_up[:, d:]   (reference.cpp:55-64)
void silu_and_mul_quant_fp8(void* q, void* scales, const void* gate_up, dtype dt, int64_t tokens,
                            int64_t d, int group_size = 128, void* stream = nullptr);

//   residual [rows, cols] dt, updated in place: residual += x
//   q [rows, cols] E4M3, scales [rows, cols/128] of rmsnorm(residual) * weight
//   (reference.cpp:23-35; eps as in the reference's default)
void fused_add_rmsnorm_quant_fp8(void* residual, void* q, void* scales, const void* x,
                                 const void* weight, dtype dt, int64_t rows, int64_t cols,
                                 float eps = 1e-6f, int group_size = 128,
                                 void* stream = nullptr);

// --- extension: the quantizer and the GEMM in one call ------------------------
// No counterpart in the reference ops.h, whose decode step is two calls:
// quant_fp8_per_token_group (ops.h:64-65) then w8a8_block_fp8_gemm
// (ops.h:81-84) on its output.  This call writes the same q / scales and the
// same C as that pair (group_size 128, the GEMM's automatic kernel choice),
// bit for bit; up to 8 rows it is one kernel launch (the GEMM quantizes its
// own activations), otherwise the two launches on the stream.
//   x: [m, k] in dt (fp32 / fp16 / bf16);  q: [m, k] E4M3;  scales: [m, k/128]
//   b_q, b_scales, c: as for w8a8_block_fp8_gemm
// Shape checks and diagnostics as for the GEMM; an invalid dt or out_dt is a
// silent no-op.
void quant_w8a8_block_fp8_gemm(void* c, void* q, void* scales, const void* x, dtype dt,
                               const void* b_q, const void* b_scales, int64_t m, int64_t n,
                               int64_t k, int group_size = 128, int block_n = 128,
                               dtype out_dt = dtype::bf16, void* stream = nullptr);

// --- extension: grouped W8A8 blockwise-FP8 GEMM over MoE experts --------------
// No counterpart in the reference ops.h: its roadmap lists the grouped GEMM
// for MoE (docs/ROADMAP.md:39, "contiguous / masked layouts"); this is the
// contiguous layout on the GEMM above.  The activation rows are sorted by
// expert: expert e owns rows [expert_offsets[e], expert_offsets[e+1]).
//   a_q: [m, k] E4M3, a_scales: [m, k/128] fp32 (as for the GEMM)
//   b_q: [num_experts, n, k] E4M3, b_scales: [num_experts, ceil(n/128), k/128]
//   expert_offsets: device int32 [num_experts + 1], non-decreasing, [0] = 0,
//                   [num_experts] = m (values are clamped to [0, m])
//   C:   [m, n] in out_dt; row r = A[r] x B[e]^T for the expert e owning r
// Shape checks and diagnostics as for the GEMM (m = 0 is a no-op).
void w8a8_block_fp8_grouped_gemm(void* c, const void* a_q, const void* a_scales,
                                 const void* b_q, const void* b_scales,
                                 const void* expert_offsets, int64_t m, int64_t n, int64_t k,
                                 int64_t num_experts, int group_size = 128, int block_n = 128,
                                 dtype out_dt = dtype::bf16, void* stream = nullptr);

// The masked layout of the same GEMM (the roadmap's second layout): every
// expert has a fixed block of max_m rows, of which masked_m[e] are valid, so
// the call's shapes do not depend on the routing (graph capture of decode).
//   a_q: [num_experts, max_m, k] E4M3, a_scales: [num_experts, max_m, k/128]
//   masked_m: device int32 [num_experts] (clamped to [0, max_m])
//   C:   [num_experts, max_m, n]; rows past an expert's count are not written
// expected_m: typical valid rows per expert, a hint for the tile choice
// (<= 0: max_m).  Shape checks as for the GEMM (max_m = 0 is a no-op).
void w8a8_block_fp8_grouped_gemm_masked(void* c, const void* a_q, const void* a_scales,
                                        const void* b_q, const void* b_scales,
                                        const void* masked_m, int64_t max_m, int64_t n, int64_t k,
                                        int64_t num_experts, int64_t expected_m = 0,
                                        int group_size = 128, int block_n = 128,
                                        dtype out_dt = dtype::bf16, void* stream = nullptr);

}  // namespace inferop
