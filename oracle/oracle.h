/* CPU oracle for the blockwise-FP8 W8A8 path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU golden path (TheonHuang/Inference,
 * `inferop` v0.1.0).  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or as the timed CPU
 * baseline; the product library never links or calls it.
 *
 * Every function cites the reference file:line it follows.  How each one is
 * pinned (golden vectors, the compiled reference, closed forms) is listed in
 * oracle.c next to it.
 */
#ifndef INFEROP_ORACLE_H
#define INFEROP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* include/inferop/fp8.h:40-59 */
float orc_e4m3_to_float(uint8_t b);
/* include/inferop/fp8.h:62-96 */
uint8_t orc_float_to_e4m3(float f);
/* include/inferop/common.h:55-61 */
float orc_bf16_to_float(uint16_t v);
uint16_t orc_float_to_bf16(float f);
/* include/inferop/common.h:63-101 */
float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);

/* reference/reference.cpp:65-80 */
void orc_quant_fp8_per_token_group(uint8_t* q, float* scales, const float* x, int64_t rows,
                                   int64_t cols, int32_t group_size);
/* reference/reference.cpp:82-91 */
void orc_dequant_fp8_per_token_group(float* x, const uint8_t* q, const float* scales,
                                     int64_t rows, int64_t cols, int32_t group_size);
/* reference/reference.cpp:93-110, whole output; (row, 64-column block) items
 * spread over OpenMP threads (per-element arithmetic and summation order
 * unchanged, so the result does not depend on the thread count). */
void orc_w8a8_block_fp8_gemm(float* c, const uint8_t* a_q, const float* a_scales,
                             const uint8_t* b_q, const float* b_scales, int64_t m, int64_t n,
                             int64_t k, int32_t group_size, int32_t block_n, int32_t threads);
/* Same, for a chosen list of output rows only: c is [nrows, n]. */
void orc_w8a8_block_fp8_gemm_rows(float* c, const uint8_t* a_q, const float* a_scales,
                                  const uint8_t* b_q, const float* b_scales, int64_t m, int64_t n,
                                  int64_t k, int32_t group_size, int32_t block_n,
                                  const int64_t* rows, int64_t nrows, int32_t threads);
/* tests/test_gemm.cpp:28-45 : per (block_n x group_size) weight block quantization. */
void orc_weight_block_quant(uint8_t* b_q, float* b_scales, const float* w, int64_t n, int64_t k,
                            int32_t group_size, int32_t block_n);

/* reference/reference.cpp:11-21 (rows x cols fp32, eps as given). */
void orc_rmsnorm(float* out, const float* in, const float* weight, int64_t rows, int64_t cols,
                 float eps);
/* reference/reference.cpp:23-35: residual += x in place, out = rmsnorm(residual). */
void orc_fused_add_rmsnorm(float* residual, float* out, const float* x, const float* weight,
                           int64_t rows, int64_t cols, float eps);
/* reference/reference.cpp:55-64: out[t, i] = silu(gate_up[t, i]) * gate_up[t, d + i]. */
void orc_silu_and_mul(float* out, const float* gate_up, int64_t tokens, int64_t d);

/* reference/reference.cpp:152-181: softmax over num_experts logits per token,
 * experts stably sorted by probability descending (index ascending on ties),
 * the first topk with weight p / l, renormalized by their sum on request. */
void orc_topk_softmax(int32_t* topk_ids, float* topk_weights, const float* logits, int64_t tokens,
                      int32_t num_experts, int32_t topk, int32_t renormalize);

/* Independent E4M3 encoder: nearest point of the 253-value finite grid built
 * from the OCP definition, ties to the even encoding, |f| >= 448 saturates
 * (tests/test_fp8.cpp:8-50 describes the same oracle).  NaN -> sign|0x7F. */
uint8_t orc_grid_encode(float f);

/* Exhaustive sweeps over the fp32 bit patterns [lo, hi) (hi <= 2^32), OpenMP
 * parallel.  Return the number of inputs where the two encoders differ. */
uint64_t orc_sweep_encode_vs_grid(uint64_t lo, uint64_t hi);
/* Order-dependent checksum of orc_float_to_e4m3 over [lo, hi):
 * sum_i code(i) * ((i * 2654435761) mod 2^32), mod 2^64. */
uint64_t orc_encode_checksum(uint64_t lo, uint64_t hi);

/* out[i - lo] = conversion of the fp32 bit pattern i, for i in [lo, hi). */
void orc_encode_range(uint64_t lo, uint64_t hi, uint8_t* out);
void orc_bf16_range(uint64_t lo, uint64_t hi, uint16_t* out);
void orc_half_range(uint64_t lo, uint64_t hi, uint16_t* out);

#ifdef __cplusplus
}
#endif

#endif
