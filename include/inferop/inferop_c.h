/* inferop (MI355X build) : C-ABI of the blockwise-FP8 W8A8 path.
 *
 * The flat, FFI-friendly form of the C++ API in inferop/ops.h (ctypes, cgo,
 * JNI or N-API bind these).  Same argument meaning and the same no-op and
 * error behaviour as the C++ functions; in addition each call returns a
 * status code.  Plain C types only: tensors are device pointers, dtypes are
 * the int32 values of inferop::dtype (0 fp32, 1 fp16, 2 bf16, 3 fp8_e4m3),
 * the stream is a hipStream_t passed as void* (NULL = null stream).
 *
 * Each entry point names the reference interface it replaces
 * (TheonHuang/Inference, include/inferop/ops.h).
 */
#ifndef INFEROP_C_H
#define INFEROP_C_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  INFEROP_OK = 0,
  INFEROP_ERR_SHAPE = 1,     /* rejected shape: the call did nothing */
  INFEROP_ERR_DTYPE = 2,     /* unsupported dtype: the call did nothing */
  INFEROP_ERR_DEVICE = 3,    /* no HIP device / unsupported architecture */
  INFEROP_ERR_LAUNCH = 4,    /* the HIP runtime reported an error */
  INFEROP_ERR_ARGUMENT = 5   /* invalid argument of a tuning entry point */
};

/* Human-readable text of a status code. */
const char* inferop_status_string(int status);

/* --- introspection: replaces ops.h:19-25 --- */
int inferop_has_device(void);                 /* has_cuda() */
int inferop_device_count(void);               /* device_count() */
const char* inferop_device_name(int ordinal); /* device_name(int) */
int inferop_device_arch(int ordinal);         /* device_sm_version(int): gfx number, e.g. 950 */

/* --- replaces ops.h:64-65 quant_fp8_per_token_group ---
 * Shapes with rows <= 0, cols <= 0, group_size <= 0 or cols % group_size != 0
 * return INFEROP_ERR_SHAPE; dt outside {fp32, fp16, bf16} returns
 * INFEROP_ERR_DTYPE; in both cases nothing is written (the reference's
 * silent no-op). */
int inferop_quant_fp8_per_token_group(void* q, void* scales, const void* x, int32_t dt,
                                      int64_t rows, int64_t cols, int32_t group_size,
                                      void* stream);

/* --- replaces ops.h:68-70 dequant_fp8_per_token_group --- same guards. */
int inferop_dequant_fp8_per_token_group(void* x, int32_t dt, const void* q, const void* scales,
                                        int64_t rows, int64_t cols, int32_t group_size,
                                        void* stream);

/* --- replaces ops.h:81-84 w8a8_block_fp8_gemm ---
 * group_size != 128, block_n != 128, k % 128 != 0, m <= 0 or n <= 0 print the
 * reference's one-line diagnostic to stderr and return INFEROP_ERR_SHAPE;
 * out_dt outside {fp32, fp16, bf16} returns INFEROP_ERR_DTYPE silently. */
int inferop_w8a8_block_fp8_gemm(void* c, const void* a_q, const void* a_scales, const void* b_q,
                                const void* b_scales, int64_t m, int64_t n, int64_t k,
                                int32_t group_size, int32_t block_n, int32_t out_dt,
                                void* stream);

/* --- allocation-free variant of inferop_w8a8_block_fp8_gemm ---
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  Same arguments, guards, kernel choice and results as
 * inferop_w8a8_block_fp8_gemm; the split-K partials and counters live in a
 * fixed device array of 64 MiB + 64 KiB per GPU (held from library load until
 * the process ends; its address is looked up on the first call on a device)
 * instead of a per-stream workspace, so no call allocates.  Limit: a shape
 * whose automatic choice needs more split-K scratch than that array returns
 * INFEROP_ERR_ARGUMENT and writes nothing (no shape does: the automatic
 * choice stays within the same capacity).  Every split-K call on one GPU
 * shares the array: such calls that overlap in time on one GPU (other
 * streams, a graph replayed beside eager calls) race and must not be issued;
 * the counters return to zero at the end of every call. */
int inferop_w8a8_block_fp8_gemm_noalloc(void* c, const void* a_q, const void* a_scales,
                                        const void* b_q, const void* b_scales, int64_t m,
                                        int64_t n, int64_t k, int32_t group_size,
                                        int32_t block_n, int32_t out_dt, void* stream);

/* --- extension: the quantizer and the GEMM in one call (no counterpart in
 * the reference; the pair quant_fp8_per_token_group, ops.h:64-65, then
 * w8a8_block_fp8_gemm, ops.h:81-84), see inferop::quant_w8a8_block_fp8_gemm
 * in ops.h.  x [m, k] in dt; q [m, k] and scales [m, k/128] receive exactly
 * what inferop_quant_fp8_per_token_group writes (group 128) and c exactly what
 * inferop_w8a8_block_fp8_gemm computes from them.  The GEMM's guards (with
 * its diagnostic, INFEROP_ERR_SHAPE) and dt / out_dt outside {fp32, fp16,
 * bf16} (INFEROP_ERR_DTYPE); nothing is written then.  One kernel launch
 * where the GEMM's automatic choice is an unsplit 8-row decode configuration
 * (m <= 8) with x 16-byte and q 8-byte aligned, else two. */
int inferop_quant_w8a8_block_fp8_gemm(void* c, void* q, void* scales, const void* x, int32_t dt,
                                      const void* b_q, const void* b_scales, int64_t m, int64_t n,
                                      int64_t k, int32_t group_size, int32_t block_n,
                                      int32_t out_dt, void* stream);
/* Kernel launches that call makes for an m x n x k problem with aligned
 * pointers (1 or 2; -1 for an invalid shape). */
int inferop_quant_w8a8_block_fp8_gemm_launches(int64_t m, int64_t n, int64_t k);

/* --- replaces ops.h:108-110 topk_softmax ---
 * tokens <= 0, num_experts <= 0, num_experts > 1024, topk <= 0 or
 * topk > num_experts return INFEROP_ERR_SHAPE and write nothing (the
 * reference's silent no-op).  renormalize: 0 or 1. */
int inferop_topk_softmax(int32_t* topk_ids, void* topk_weights, const void* logits, int32_t tokens,
                         int32_t num_experts, int32_t topk, int32_t renormalize, void* stream);

/* --- extension: 128x128 weight block quantizer (no counterpart in the
 * reference ops.h; the recipe of its tests/test_gemm.cpp:28-45), see
 * inferop::quant_fp8_weight_block in ops.h.  group_size != 128,
 * block_n != 128, n <= 0, k <= 0 or k % 128 != 0 return INFEROP_ERR_SHAPE;
 * dt outside {fp32, fp16, bf16} INFEROP_ERR_DTYPE; w not 16-byte or b_q not
 * 8-byte aligned INFEROP_ERR_ARGUMENT; nothing is written in those cases. */
int inferop_quant_fp8_weight_block(void* b_q, void* b_scales, const void* w, int32_t dt, int64_t n,
                                   int64_t k, int32_t group_size, int32_t block_n, void* stream);

/* --- extension: producers fused with the per-token-group quantizer (no
 * counterparts in the reference ops.h; see inferop::silu_and_mul_quant_fp8 and
 * inferop::fused_add_rmsnorm_quant_fp8 in ops.h).  group_size != 128,
 * tokens/rows <= 0, d/cols <= 0 or not a multiple of 128 return
 * INFEROP_ERR_SHAPE; dt outside {fp32, fp16, bf16} INFEROP_ERR_DTYPE; a dt
 * tensor not 16-byte aligned or q not 8-byte aligned INFEROP_ERR_ARGUMENT. */
int inferop_silu_and_mul_quant_fp8(void* q, void* scales, const void* gate_up, int32_t dt,
                                   int64_t tokens, int64_t d, int32_t group_size, void* stream);
int inferop_fused_add_rmsnorm_quant_fp8(void* residual, void* q, void* scales, const void* x,
                                        const void* weight, int32_t dt, int64_t rows, int64_t cols,
                                        float eps, int32_t group_size, void* stream);

/* --- extension: grouped blockwise-FP8 GEMM over MoE experts (no counterpart
 * in the reference's ops.h; its roadmap lists it, docs/ROADMAP.md:39) ---
 * Contiguous layout, as inferop::w8a8_block_fp8_grouped_gemm in ops.h:
 * a_q [m, k] rows sorted by expert, expert e owning rows
 * [expert_offsets[e], expert_offsets[e+1]) (device int32, num_experts + 1
 * entries, clamped to [0, m] on the device); b_q [num_experts, n, k];
 * b_scales [num_experts, ceil(n/128), k/128]; c [m, n].  The GEMM's shape
 * rules (INFEROP_ERR_SHAPE with its diagnostic) plus num_experts >= 1 and
 * m >= 0; m = 0 returns INFEROP_OK without a launch. */
int inferop_w8a8_block_fp8_grouped_gemm(void* c, const void* a_q, const void* a_scales,
                                        const void* b_q, const void* b_scales,
                                        const int32_t* expert_offsets, int64_t m, int64_t n,
                                        int64_t k, int64_t num_experts, int32_t group_size,
                                        int32_t block_n, int32_t out_dt, void* stream);
/* Masked layout, as inferop::w8a8_block_fp8_grouped_gemm_masked in ops.h:
 * a_q [num_experts, max_m, k], masked_m device int32 [num_experts] valid rows
 * per expert (clamped to [0, max_m]), c [num_experts, max_m, n] (rows past a
 * count are not written); expected_m: tile-choice hint (<= 0: max_m).
 * max_m = 0 returns INFEROP_OK without a launch. */
int inferop_w8a8_block_fp8_grouped_gemm_masked(void* c, const void* a_q, const void* a_scales,
                                               const void* b_q, const void* b_scales,
                                               const int32_t* masked_m, int64_t max_m, int64_t n,
                                               int64_t k, int64_t num_experts, int64_t expected_m,
                                               int32_t group_size, int32_t block_n,
                                               int32_t out_dt, void* stream);

/* --- tuning and testing (no counterpart in the reference) ---
 * The GEMM with an explicit kernel configuration and split-K factor instead
 * of the automatic gfx950 choice.  config in [0, inferop_gemm_num_configs()).
 * The persistent configurations ("per_" names) cut the tiles of their last,
 * partial round into split_k K ranges and need an even K / 128; other K
 * return INFEROP_ERR_ARGUMENT.  A split whose partials exceed a workspace
 * slot, or on a stream that can take no slot, returns INFEROP_ERR_ARGUMENT. */
int inferop_gemm_num_configs(void);
const char* inferop_gemm_config_name(int config);
int inferop_w8a8_block_fp8_gemm_config(void* c, const void* a_q, const void* a_scales,
                                       const void* b_q, const void* b_scales, int64_t m,
                                       int64_t n, int64_t k, int32_t out_dt, int32_t config,
                                       int32_t split_k, void* stream);
/* The configuration and split-K factor the automatic choice would use (on a
 * stream that has, or can still take, a split-K workspace slot). */
int inferop_gemm_select(int64_t m, int64_t n, int64_t k, int32_t* config, int32_t* split_k);
/* Split-K workspace of the current device: a fixed pool of *slots_total
 * slots of *slot_bytes each (fp32 partials plus arrival counters), of which
 * *slots_used are held by streams.  A stream takes a slot at its first
 * split-K call and keeps it until the process ends; once all are held, the
 * automatic choice runs later streams' GEMMs unsplit and
 * inferop_w8a8_block_fp8_gemm_config with a split returns
 * INFEROP_ERR_ARGUMENT on them.  Any pointer may be NULL. */
int inferop_splitk_workspace_info(int32_t* slots_used, int32_t* slots_total, int64_t* slot_bytes);
/* The grouped GEMM with an explicit configuration: one of the tiled
 * configurations with a grouped variant (others return INFEROP_ERR_ARGUMENT);
 * and the configuration the automatic choice would use. */
int inferop_w8a8_block_fp8_grouped_gemm_config(void* c, const void* a_q, const void* a_scales,
                                               const void* b_q, const void* b_scales,
                                               const int32_t* expert_offsets, int64_t m,
                                               int64_t n, int64_t k, int64_t num_experts,
                                               int32_t out_dt, int32_t config, void* stream);
int inferop_grouped_gemm_select(int64_t m, int64_t n, int64_t k, int64_t num_experts,
                                int32_t* config);
/* The configuration the masked grouped GEMM would choose for these
 * arguments (expected_m as in inferop_w8a8_block_fp8_grouped_gemm_masked). */
int inferop_grouped_gemm_masked_select(int64_t max_m, int64_t n, int64_t k, int64_t num_experts,
                                       int64_t expected_m, int32_t* config);
int inferop_w8a8_block_fp8_grouped_gemm_masked_config(void* c, const void* a_q,
                                                      const void* a_scales, const void* b_q,
                                                      const void* b_scales,
                                                      const int32_t* masked_m, int64_t max_m,
                                                      int64_t n, int64_t k, int64_t num_experts,
                                                      int32_t out_dt, int32_t config,
                                                      void* stream);

/* --- diagnostics (no counterpart in the reference) ---
 * Compares, on the current device, the hardware E4M3 conversions the fast
 * paths use with the reference-semantics software codec, for every fp32 bit
 * pattern in [lo, hi) (hi <= 2^32).  counts: 4 device uint64, zeroed by the
 * caller: [0] mismatches inside the quantizer fast-path domain (finite,
 * |v| < 464), [1] mismatches outside it, [2] checksum of the software codes,
 * [3] decode mismatches over the 256 bytes. */
int inferop_selftest_fp8_codec(uint64_t lo, uint64_t hi, uint64_t* counts, void* stream);

/* --- measurement kernels (no counterpart in the reference) ---
 * The ceilings the bench holds the path's kernels against, on the current
 * device.  inferop_diag_read_stream reads `bytes` (a multiple of 16, >= 16)
 * from the device buffer src once with `blocks` workgroups of 256 lanes
 * (16-byte non-temporal loads, four in flight per lane): a GEMM that streams
 * the same bytes cannot take less time.  inferop_diag_mfma_loop runs `blocks`
 * workgroups of 4 waves, each wave issuing iters x 32 E4M3 MFMAs of 16x16x128
 * (65536 flops each; one wave's share of a 256x256 tile per scale group) from
 * registers, with promote != 0 also the four fp32
 * scale-promotion FMAs per MFMA of the blockwise GEMM: the matrix-core rate
 * the chip sustains without memory traffic.  sink: one device uint32 of
 * scratch. */
int inferop_diag_read_stream(const void* src, int64_t bytes, int32_t blocks, void* sink,
                             void* stream);
int inferop_diag_mfma_loop(int32_t iters, int32_t blocks, int32_t promote, void* sink,
                           void* stream);
/* inferop_diag_stripe_read reads the [n, k] byte matrix b once with one
 * workgroup of 8 waves per 16-row stripe (the decode GEMM's unit of work),
 * every load of a workgroup in flight at once, in access pattern `pattern`:
 * 0 register loads of 8 rows x 128 B per instruction, 1 register loads of
 * 1 KB contiguous, 2 register loads in the MFMA operand layout (16 rows x 64 B
 * per instruction), 3 direct global->LDS loads of 8 rows x 128 B (the decode
 * kernels' loads), 4 pattern 0's register loads written to LDS with
 * ds_write_b128 in pattern 3's layout.  stripes > 0: workgroup i reads stripe i % stripes, so the
 * data is L2-resident and the launch measures a compute unit's load rate.
 * n a multiple of 16, k / 1024 in {2, 7, 8}; sink: one device uint32. */
int inferop_diag_stripe_read(const void* b, int64_t n, int64_t k, int32_t pattern,
                             int32_t stripes, void* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif
