/* Thin internal C-ABI between the C++ front end (ops.cpp, built with g++ and
 * no HIP headers) and the HIP translation units (built with hipcc for
 * gfx950).  Plain C types only; every launch function returns a hipError_t
 * value as int (0 = hipSuccess).  Arguments are assumed validated by the
 * caller (shapes, dtypes); the launch functions only check what the kernels
 * themselves assume (alignment, grid limits). */
#ifndef INFEROP_HIP_LAUNCH_H
#define INFEROP_HIP_LAUNCH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- device introspection ---- */
int inferop_hip_device_count(void);
/* name (NUL-terminated, truncated to name_len), arch number (the gfx digits
 * read as hexadecimal: gfx950 -> 0x950),
 * CU count.  Returns hipError_t. */
int inferop_hip_device_info(int ordinal, char* name, int name_len, int* arch, int* cu_count);
int inferop_hip_current_device(int* ordinal);

/* ---- quantizer / dequantizer (dt: 0 fp32, 1 fp16, 2 bf16) ---- */
int inferop_hip_quant_fp8_group(void* q, float* scales, const void* x, int32_t dt, int64_t rows,
                                int64_t cols, int32_t group_size, void* stream);
int inferop_hip_dequant_fp8_group(void* x, int32_t dt, const uint8_t* q, const float* scales,
                                  int64_t rows, int64_t cols, int32_t group_size, void* stream);
/* 128 x 128 weight blocks of w [n, k] (k % 128 == 0); w 16-byte, q 8-byte
 * aligned (hipErrorInvalidValue otherwise). */
int inferop_hip_weight_block_quant(uint8_t* q, float* scales, const void* w, int32_t dt, int64_t n,
                                   int64_t k, void* stream);

/* ---- fused producers + quantizer (d, cols multiples of 128; dt inputs
 * 16-byte aligned, q 8-byte aligned) ---- */
int inferop_hip_silu_mul_quant(uint8_t* q, float* scales, const void* gate_up, int32_t dt,
                               int64_t tokens, int64_t d, void* stream);
int inferop_hip_add_rmsnorm_quant(void* residual, uint8_t* q, float* scales, const void* x,
                                  const void* weight, int32_t dt, int64_t rows, int64_t cols,
                                  float eps, void* stream);

/* ---- MoE routing: softmax + top-k per token (num_experts <= 1024) ---- */
int inferop_hip_topk_softmax(int32_t* ids, float* weights, const float* logits, int tokens,
                             int num_experts, int topk, int renormalize, void* stream);

/* ---- blockwise FP8 GEMM ----
 * cfg: index into the kernel table (inferop_hip_gemm_num_configs());
 * split_k: number of K partitions (1 = none); partitions > 1 reduce through
 * a library-owned fp32 workspace with a last-arriving-block fixup. */
typedef struct {
  int32_t cfg;
  int32_t split_k;
} inferop_gemm_launch;

typedef struct {
  int32_t bn;     /* block tile along N */
  int32_t bm;     /* block tile along M */
  int32_t waves;  /* waves per workgroup */
  int32_t kind;   /* 1 = decode (16-row weight stripes), 2 = LDS-staged output tiles,
                     3 = persistent LDS-staged tiles (K/128 even; split_k > 1 cuts
                         the tiles of the last, partial round along K),
                     4 = wide decode: bn weight rows over all of K (or one of split_k
                         K ranges) with bm activation rows */
  const char* name;
  int32_t grouped; /* kind 2: has a grouped-expert variant */
} inferop_gemm_cfg_info;

/* Capacity of one split-K workspace slot: fp32 partial bytes and arrival
 * counters (one per output tile).  A launch whose split needs more is
 * rejected with hipErrorInvalidValue.  Each device has
 * INFEROP_SPLITK_WS_SLOTS slots, handed out one per stream at the stream's
 * first split-K call and kept by it until the process ends. */
#define INFEROP_SPLITK_WS_BYTES (64ll << 20)
#define INFEROP_SPLITK_WS_COUNTERS 16384
#define INFEROP_SPLITK_WS_SLOTS 8

/* Takes (or finds) the current device's workspace slot of `stream`, allocating
 * it on the stream's first use.  0 on success; hipErrorOutOfMemory when every
 * slot belongs to another stream (the caller then launches unsplit). */
int inferop_hip_splitk_reserve(void* stream);
/* Slots of the current device handed out so far. */
int inferop_hip_splitk_slots_used(void);

int inferop_hip_gemm_num_configs(void);
int inferop_hip_gemm_config_info(int32_t cfg, inferop_gemm_cfg_info* info);
/* Split-K workspace bytes a launch of cfg with split_k partitions needs for
 * an m x n output (0 when it splits nothing; -1 for an invalid configuration
 * or more output tiles than counters).  The split is clamped to k / 128 as
 * the launch clamps it. */
int64_t inferop_hip_gemm_workspace_bytes(int32_t cfg, int32_t split_k, int64_t m, int64_t n,
                                         int64_t k);
int inferop_hip_gemm_w8a8_block(void* c, const uint8_t* a_q, const float* a_scales,
                                const uint8_t* b_q, const float* b_scales, int64_t m, int64_t n,
                                int64_t k, int32_t out_dt, const inferop_gemm_launch* launch,
                                void* stream);

/* Same launch without any allocation: split-K partials and counters come
 * from a file-scope device array of INFEROP_SPLITK_WS_BYTES +
 * 4 * INFEROP_SPLITK_WS_COUNTERS bytes per GPU (its address looked up with
 * hipGetSymbolAddress on the first call on a device, which also zeroes the
 * counters on that call's stream).  Calls on one GPU share it. */
int inferop_hip_gemm_w8a8_block_noalloc(void* c, const uint8_t* a_q, const float* a_scales,
                                        const uint8_t* b_q, const float* b_scales, int64_t m,
                                        int64_t n, int64_t k, int32_t out_dt,
                                        const inferop_gemm_launch* launch, void* stream);

/* The quantizer (group 128) fused with the decode GEMM, one launch: x [m, k]
 * in dt (fp32 / fp16 / bf16, 16-byte aligned) is quantized exactly as
 * inferop_hip_quant_fp8_group would (q [m, k] 8-byte aligned, qs [m, k/128])
 * and C [m, n] = GEMM(q, qs, b_q, b_scales) exactly as the 8-row wide decode
 * configuration with `waves` waves (4 or 8) computes it.  1 <= m <= 8 and at
 * most 8 scale groups per wave (k / 128 <= 8 * waves); other calls return
 * hipErrorInvalidValue without a launch. */
int inferop_hip_quant_gemm_decode(void* c, uint8_t* q, float* qs, const void* x, int32_t dt,
                                  const uint8_t* b_q, const float* b_scales, int64_t m, int64_t n,
                                  int64_t k, int32_t out_dt, int32_t waves, void* stream);

/* Grouped (MoE expert) GEMM; B [experts, n, k], b_scales [experts,
 * ceil(n/128), k/128]; C [m, n]; cfg must be a tiled configuration with a
 * grouped variant (inferop_gemm_cfg_info.grouped).
 * max_m == 0, contiguous layout: A [m, k] rows sorted by expert, expert e
 * owning rows [offsets[e], offsets[e+1]) (offsets: device int32
 * [experts + 1], clamped to [0, m] on the device).
 * max_m > 0, masked layout: m == experts * max_m, expert e owning rows
 * [e * max_m, e * max_m + offsets[e]) (offsets: device int32 [experts] valid
 * counts, clamped to [0, max_m]); other rows of C are not written. */
int inferop_hip_gemm_w8a8_block_grouped(void* c, const uint8_t* a_q, const float* a_scales,
                                        const uint8_t* b_q, const float* b_scales,
                                        const int32_t* offsets, int64_t m, int64_t n, int64_t k,
                                        int64_t experts, int64_t max_m, int32_t out_dt,
                                        int32_t cfg, void* stream);

/* ---- measurement kernels for the bench's ceilings ----
 * read_stream: one plain read of `bytes` (a multiple of 16) from src by
 * `blocks` workgroups of 256 lanes; sink: one device uint32 of scratch.
 * mfma_loop: `blocks` workgroups of 4 waves, each wave issuing iters x 32
 * E4M3 MFMAs of 16x16x128 from registers (65536 flops each; one wave's share
 * of a 256x256 tile per scale group), with promote the four scale-promotion
 * FMAs per MFMA the GEMM adds. */
int inferop_hip_diag_read_stream(const void* src, int64_t bytes, int32_t blocks, uint32_t* sink,
                                 void* stream);
int inferop_hip_diag_mfma_loop(int32_t iters, int32_t blocks, int32_t promote, uint32_t* sink,
                               void* stream);
/* stripe_read: one read of the [n, k] byte matrix b by one 8-wave workgroup
 * per 16-row stripe, all of a workgroup's loads in flight, in access pattern
 * 0-4 (8-row register loads, contiguous register loads, MFMA-layout register
 * loads, 8-row direct-to-LDS loads, 8-row register loads written to LDS);
 * stripes > 0 makes workgroup i read
 * stripe i % stripes (L2-resident).  n % 16 == 0, k / 1024 in {2, 7, 8}. */
int inferop_hip_diag_stripe_read(const void* b, int64_t n, int64_t k, int32_t pattern,
                                 int32_t stripes, uint32_t* sink, void* stream);

/* ---- device self-test of the E4M3 conversions used by the fast paths ----
 * counts[0]: fp32 patterns in [lo, hi) inside the quantizer fast-path domain
 *            (finite, |v| < 464) where the hardware encode differs from the
 *            software (reference-semantics) encode;
 * counts[1]: same, outside that domain (informational);
 * counts[2]: checksum sum_i sw_encode(i) * ((i * 2654435761) mod 2^32);
 * counts[3]: bytes 0..255 whose hardware decode differs from the software
 *            decode (bitwise, NaNs compared as NaN).
 * counts must point to 4 device uint64 zero-initialised by the caller. */
int inferop_hip_selftest_fp8_codec(uint64_t lo, uint64_t hi, uint64_t* counts, void* stream);

#ifdef __cplusplus
}
#endif

#endif
