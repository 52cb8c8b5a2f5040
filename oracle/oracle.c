/* CPU oracle for the blockwise-FP8 W8A8 path -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates, step by step, the reference's CPU golden code (paths relative to
 * the reference repository TheonHuang/Inference):
 *   include/inferop/fp8.h:40-96       E4M3 decode / encode
 *   include/inferop/common.h:55-101   bf16 / fp16 host conversions
 *   reference/reference.cpp:65-110    quantizer, dequantizer, GEMM
 *   tests/test_gemm.cpp:28-45         weight block quantizer of the GEMM tests
 *
 * Pinning (what makes a mistake here fail a test):
 *   - codec: exhaustive 2^32 comparison with orc_grid_encode (an independent
 *     nearest-grid-point encoder) and with the compiled reference; the decode
 *     of all 256 bytes against the OCP closed form; the reference's edge and
 *     tie list (tests/test_fp8.cpp:75-91).
 *   - bf16 / fp16: exhaustive comparison with the compiled reference and with
 *     numpy's IEEE conversions outside the two documented fp16 departures.
 *   - quantizer / dequantizer / GEMM: byte- and bit-exact comparison with the
 *     compiled reference on seeded cases and the committed golden fixtures; the
 *     zero-group known answer (tests/test_quant.cpp:34-41); the GEMM against a
 *     float64 numpy matmul of the dequantized operands, linearity in the
 *     scales, and invariance under a permutation of K inside one group.
 *
 * x86-64 note: the reference runs on x86-64, where an invalid operation (0/0,
 * Inf/Inf) produces the negative default NaN; the quantizer's bytes for such
 * groups therefore carry the sign bit.  This file is compiled for the same
 * host and inherits the same behaviour.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t bits_of(float f) {
  uint32_t w;
  memcpy(&w, &f, 4);
  return w;
}
static inline float float_of(uint32_t w) {
  float f;
  memcpy(&f, &w, 4);
  return f;
}

/* fp8.h:40-59 : sign, 4-bit exponent, 3-bit mantissa; S.1111.111 is NaN;
 * E == 0 is m * 2^-9, renormalised onto the fp32 grid by shifting m up. */
float orc_e4m3_to_float(uint8_t b) {
  uint32_t s = (uint32_t)(b >> 7) << 31;
  uint32_t E = ((uint32_t)b >> 3) & 0xFu;
  uint32_t m = (uint32_t)b & 0x7u;
  if (E == 15u && m == 7u) return float_of(0x7FC00000u | s);
  if (E == 0u) {
    if (m == 0u) return float_of(s);
    uint32_t mm = m;
    int e32 = 121;
    while (mm < 8u) {
      mm <<= 1;
      --e32;
    }
    return float_of(s | ((uint32_t)e32 << 23) | ((mm & 7u) << 20));
  }
  return float_of(s | ((E + 120u) << 23) | (m << 20));
}

/* fp8.h:62-96 : integer RNE with SATFINITE. */
uint8_t orc_float_to_e4m3(float f) {
  uint32_t x = bits_of(f);
  uint32_t sign = (x >> 24) & 0x80u;
  uint32_t a = x & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint8_t)(sign | 0x7Fu);  /* :66 NaN */
  if (a == 0x7F800000u) return (uint8_t)(sign | 0x7Eu); /* :67 Inf -> 448 */
  int e = (int)((a >> 23) & 0xFFu) - 127;
  if (e >= 9) return (uint8_t)(sign | 0x7Eu); /* :69 */
  if (e >= -6) {                              /* :70-83 normal */
    uint32_t man = (a & 0x7FFFFFu) | 0x800000u;
    uint32_t keep = man >> 20;
    uint32_t rem = man & 0xFFFFFu;
    uint32_t r = (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) ? 1u : 0u;
    uint32_t mq = keep - 8u + r;
    uint32_t E = (uint32_t)(e + 7);
    if (mq == 8u) {
      mq = 0;
      E += 1u;
    }
    if (E >= 16u || (E == 15u && mq == 7u)) return (uint8_t)(sign | 0x7Eu);
    return (uint8_t)(sign | (E << 3) | mq);
  }
  if (e >= -10) { /* :84-94 subnormal band */
    uint32_t man = (a & 0x7FFFFFu) | 0x800000u;
    uint32_t sh = (uint32_t)(14 - e);
    uint32_t keep = man >> sh;
    uint32_t rem = man & ((1u << sh) - 1u);
    uint32_t half = 1u << (sh - 1);
    uint32_t r = (rem > half || (rem == half && (keep & 1u))) ? 1u : 0u;
    uint32_t md = keep + r;
    if (md == 8u) return (uint8_t)(sign | 0x08u);
    return (uint8_t)(sign | md);
  }
  return (uint8_t)sign; /* :95 */
}

/* common.h:55 */
float orc_bf16_to_float(uint16_t v) { return float_of((uint32_t)v << 16); }

/* common.h:57-61 : x + 0x7FFF + lsb, no NaN special case. */
uint16_t orc_float_to_bf16(float f) {
  uint32_t x = bits_of(f);
  return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

/* common.h:63-78 */
float orc_half_to_float(uint16_t h) {
  uint32_t sign = ((uint32_t)h >> 15) & 1u;
  uint32_t ex = ((uint32_t)h >> 10) & 0x1Fu;
  uint32_t man = (uint32_t)h & 0x3FFu;
  float v;
  if (ex == 0) {
    if (man == 0) return sign ? -0.0f : 0.0f;
    v = ldexpf((float)man, -24);
  } else if (ex == 31) {
    if (man != 0) return nanf("");
    v = INFINITY;
  } else {
    v = ldexpf((float)(1024u + man), (int)ex - 25);
  }
  return sign ? -v : v;
}

/* common.h:80-101 (frexp / nearbyint formulation, kept as in the reference). */
uint16_t orc_float_to_half(float f) {
  if (isnan(f)) return 0x7E00;
  int neg = signbit(f) ? 1 : 0;
  float a = neg ? -f : f;
  if (isinf(a) || a > 65504.0f) return neg ? (uint16_t)0xFC00 : (uint16_t)0x7C00;
  if (a < 5.9604645e-8f) return neg ? (uint16_t)0x8000 : (uint16_t)0x0000;
  int e = 0;
  float frac = frexpf(a, &e);
  if (e < -13) {
    uint32_t m = (uint32_t)nearbyintf(ldexpf(a, 24));
    if (m >= 1024u) return neg ? (uint16_t)0x8400 : (uint16_t)0x0400;
    return (uint16_t)((neg ? 0x8000u : 0u) | m);
  }
  uint32_t m = (uint32_t)(nearbyintf(ldexpf(frac, 11)) - 1024);
  uint32_t ex = (uint32_t)(e - 1 + 15);
  if (m == 1024u) {
    m = 0;
    ex += 1;
  }
  if (ex >= 31u) return neg ? (uint16_t)0xFC00 : (uint16_t)0x7C00;
  return (uint16_t)((neg ? 0x8000u : 0u) | (ex << 10) | m);
}

/* reference.cpp:65-80 : per (row, group): absmax with std::max semantics
 * (a NaN element never replaces the running max), scale = absmax * fl32(1/448)
 * or 1 for an all-zero group, q = encode(x / scale) with IEEE division. */
void orc_quant_fp8_per_token_group(uint8_t* q, float* scales, const float* x, int64_t rows,
                                   int64_t cols, int32_t group_size) {
  const int64_t gpr = cols / group_size;
  const float inv448 = 1.0f / 448.0f;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < gpr; ++g) {
      const float* gx = x + r * cols + g * group_size;
      float absmax = 0.0f;
      for (int32_t i = 0; i < group_size; ++i) {
        float v = fabsf(gx[i]);
        absmax = (absmax < v) ? v : absmax; /* std::max(absmax, v) */
      }
      float scale = (absmax == 0.0f) ? 1.0f : absmax * inv448;
      scales[r * gpr + g] = scale;
      for (int32_t i = 0; i < group_size; ++i) {
        volatile float qv = gx[i] / scale;
        q[r * cols + g * group_size + i] = orc_float_to_e4m3(qv);
      }
    }
  }
}

/* reference.cpp:82-91 */
void orc_dequant_fp8_per_token_group(float* x, const uint8_t* q, const float* scales,
                                     int64_t rows, int64_t cols, int32_t group_size) {
  const int64_t gpr = cols / group_size;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c)
      x[r * cols + c] = orc_e4m3_to_float(q[r * cols + c]) * scales[r * gpr + c / group_size];
}

/* reference.cpp:99-108 for output row mi, columns [n0, n1). */
static void gemm_cols(float* crow, int64_t mi, const uint8_t* a_q, const float* a_scales,
                      const uint8_t* b_q, const float* b_scales, int64_t n0, int64_t n1,
                      int64_t k, int32_t group_size, int32_t block_n) {
  const int64_t kg = k / group_size;
  for (int64_t ni = n0; ni < n1; ++ni) {
    double acc = 0.0;
    for (int64_t ki = 0; ki < k; ++ki) {
      float sa = a_scales[mi * kg + ki / group_size];
      float sb = b_scales[(ni / block_n) * kg + ki / group_size];
      float av = orc_e4m3_to_float(a_q[mi * k + ki]) * sa;
      float bv = orc_e4m3_to_float(b_q[ni * k + ki]) * sb;
      acc += (double)av * (double)bv;
    }
    crow[ni] = (float)acc;
  }
}

/* Work items are (output row, 64-column block): every element still sums its
 * k products in the reference's order, so any thread count gives the same
 * bits; the column blocks let one-row products use every thread. */
#define ORC_COLS 64

void orc_w8a8_block_fp8_gemm(float* c, const uint8_t* a_q, const float* a_scales,
                             const uint8_t* b_q, const float* b_scales, int64_t m, int64_t n,
                             int64_t k, int32_t group_size, int32_t block_n, int32_t threads) {
  const int64_t nc = (n + ORC_COLS - 1) / ORC_COLS;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
  for (int64_t w = 0; w < m * nc; ++w) {
    const int64_t mi = w / nc, n0 = (w % nc) * ORC_COLS;
    gemm_cols(c + mi * n, mi, a_q, a_scales, b_q, b_scales, n0,
              n0 + ORC_COLS < n ? n0 + ORC_COLS : n, k, group_size, block_n);
  }
  (void)threads;
}

void orc_w8a8_block_fp8_gemm_rows(float* c, const uint8_t* a_q, const float* a_scales,
                                  const uint8_t* b_q, const float* b_scales, int64_t m, int64_t n,
                                  int64_t k, int32_t group_size, int32_t block_n,
                                  const int64_t* rows, int64_t nrows, int32_t threads) {
  (void)m;
  const int64_t nc = (n + ORC_COLS - 1) / ORC_COLS;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
  for (int64_t w = 0; w < nrows * nc; ++w) {
    const int64_t i = w / nc, n0 = (w % nc) * ORC_COLS;
    gemm_cols(c + i * n, rows[i], a_q, a_scales, b_q, b_scales, n0,
              n0 + ORC_COLS < n ? n0 + ORC_COLS : n, k, group_size, block_n);
  }
  (void)threads;
}

/* tests/test_gemm.cpp:28-45 : absmax over the block, scale = absmax*fl32(1/448)
 * (1 for a zero block), q = encode(w * fl32(1/scale)) -- the multiply by the
 * reciprocal is the reference test's own choice for weights. */
void orc_weight_block_quant(uint8_t* b_q, float* b_scales, const float* w, int64_t n, int64_t k,
                            int32_t group_size, int32_t block_n) {
  const int64_t nb_count = (n + block_n - 1) / block_n;
  const int64_t kg = k / group_size;
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(static)
#endif
  for (int64_t nb = 0; nb < nb_count; ++nb) {
    for (int64_t g = 0; g < kg; ++g) {
      const int64_t n_end = (nb + 1) * block_n < n ? (nb + 1) * block_n : n;
      float absmax = 0.0f;
      for (int64_t r = nb * block_n; r < n_end; ++r)
        for (int64_t i = 0; i < group_size; ++i) {
          float v = fabsf(w[r * k + g * group_size + i]);
          absmax = (absmax < v) ? v : absmax;
        }
      float scale = (absmax == 0.0f) ? 1.0f : absmax * (1.0f / 448.0f);
      b_scales[nb * kg + g] = scale;
      float inv = 1.0f / scale;
      for (int64_t r = nb * block_n; r < n_end; ++r)
        for (int64_t i = 0; i < group_size; ++i)
          b_q[r * k + g * group_size + i] = orc_float_to_e4m3(w[r * k + g * group_size + i] * inv);
    }
  }
}

/* ---- producers of the quantizer's input (the layers before each GEMM) ----
 * reference/reference.cpp:11-21, 23-35 and 55-64, loop for loop: the
 * sum of squares runs left to right in fp32, the inverse RMS is
 * 1 / sqrtf(ss / cols + eps), the scaling is (x * inv) * w, and SiLU is
 * g / (1 + expf(-g)) with the C library's expf (the function std::exp(float)
 * calls on this host).  Pinned against the compiled reference bit for bit. */
void orc_rmsnorm(float* out, const float* in, const float* weight, int64_t rows, int64_t cols,
                 float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = in + r * cols;
    float* y = out + r * cols;
    float ss = 0.0f;
    for (int64_t c = 0; c < cols; ++c) ss += x[c] * x[c];
    const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
    for (int64_t c = 0; c < cols; ++c) y[c] = x[c] * inv * weight[c];
  }
}

void orc_fused_add_rmsnorm(float* residual, float* out, const float* x, const float* weight,
                           int64_t rows, int64_t cols, float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    float* res = residual + r * cols;
    float* y = out + r * cols;
    const float* xr = x + r * cols;
    for (int64_t c = 0; c < cols; ++c) res[c] += xr[c];
    float ss = 0.0f;
    for (int64_t c = 0; c < cols; ++c) ss += res[c] * res[c];
    const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
    for (int64_t c = 0; c < cols; ++c) y[c] = res[c] * inv * weight[c];
  }
}

void orc_silu_and_mul(float* out, const float* gate_up, int64_t tokens, int64_t d) {
  for (int64_t t = 0; t < tokens; ++t) {
    const float* row = gate_up + t * 2 * d;
    for (int64_t i = 0; i < d; ++i) {
      const float g = row[i];
      out[t * d + i] = (g / (1.0f + expf(-g))) * row[d + i];
    }
  }
}

/* reference/reference.cpp:152-181.  The reference's std::stable_sort with
 * the comparator (p[a] > p[b], then a < b) is restated as a stable insertion
 * sort with the same comparator (the order is total for NaN-free logits, so
 * any stable sort gives the same permutation). */
void orc_topk_softmax(int32_t* topk_ids, float* topk_weights, const float* logits, int64_t tokens,
                      int32_t num_experts, int32_t topk, int32_t renormalize) {
  float probs[1024];
  int order[1024];
  for (int64_t t = 0; t < tokens; ++t) {
    const float* row = logits + t * num_experts;
    float mx = -INFINITY;
    for (int e = 0; e < num_experts; ++e) mx = (mx < row[e]) ? row[e] : mx;
    float l = 0.0f;
    for (int e = 0; e < num_experts; ++e) {
      probs[e] = expf(row[e] - mx);
      l += probs[e];
    }
    for (int e = 0; e < num_experts; ++e) {
      /* insert e after every element that precedes it */
      int pos = e;
      while (pos > 0) {
        const int o = order[pos - 1];
        const int before = (probs[e] != probs[o]) ? (probs[e] > probs[o]) : (e < o);
        if (!before) break;
        order[pos] = o;
        --pos;
      }
      order[pos] = e;
    }
    float wsum = 0.0f;
    for (int k = 0; k < topk; ++k) {
      topk_ids[t * topk + k] = order[k];
      topk_weights[t * topk + k] = probs[order[k]] / l;
      wsum += probs[order[k]] / l;
    }
    if (renormalize && wsum > 0.0f) {
      for (int k = 0; k < topk; ++k) topk_weights[t * topk + k] /= wsum;
    }
  }
}

/* ---- independent encoder: nearest OCP grid point ------------------------- */

/* Positive finite E4M3 values, codes 0x00..0x7E, from the OCP definition
 * (value = (1 + m/8) 2^(E-7) for E > 0, m 2^-9 for E == 0). */
static double g_grid[127];
static int g_grid_ready = 0;

static void build_grid(void) {
  for (int b = 0; b < 127; ++b) {
    int E = (b >> 3) & 0xF, m = b & 7;
    g_grid[b] = (E == 0) ? (double)m * ldexp(1.0, -9) : (1.0 + m / 8.0) * ldexp(1.0, E - 7);
  }
  g_grid_ready = 1;
}

uint8_t orc_grid_encode(float f) {
  if (!g_grid_ready) build_grid();
  uint32_t sign = (bits_of(f) >> 24) & 0x80u;
  if (isnan(f)) return (uint8_t)(sign | 0x7F);
  double a = fabs((double)f);
  if (a >= 448.0) return (uint8_t)(sign | 0x7E);
  /* the grid is increasing: find the last point <= a by bisection */
  int lo = 0, hi = 126;
  while (lo < hi) {
    int mid = (lo + hi + 1) / 2;
    if (g_grid[mid] <= a) lo = mid;
    else hi = mid - 1;
  }
  int best = lo;
  if (lo < 126) {
    double dlo = a - g_grid[lo], dhi = g_grid[lo + 1] - a;
    if (dhi < dlo || (dhi == dlo && ((lo + 1) & 1) == 0)) best = lo + 1;
  }
  return (uint8_t)(sign | (uint32_t)best);
}

uint64_t orc_sweep_encode_vs_grid(uint64_t lo, uint64_t hi) {
  if (!g_grid_ready) build_grid();
  uint64_t bad = 0;
#ifdef _OPENMP
#pragma omp parallel for reduction(+ : bad) schedule(static)
#endif
  for (int64_t i = (int64_t)lo; i < (int64_t)hi; ++i) {
    float f = float_of((uint32_t)i);
    if (orc_float_to_e4m3(f) != orc_grid_encode(f)) ++bad;
  }
  return bad;
}

uint64_t orc_encode_checksum(uint64_t lo, uint64_t hi) {
  uint64_t sum = 0;
#ifdef _OPENMP
#pragma omp parallel for reduction(+ : sum) schedule(static)
#endif
  for (int64_t i = (int64_t)lo; i < (int64_t)hi; ++i) {
    uint32_t w = (uint32_t)((uint64_t)i * 2654435761u);
    sum += (uint64_t)orc_float_to_e4m3(float_of((uint32_t)i)) * (uint64_t)w;
  }
  return sum;
}

/* Range helpers for exhaustive comparisons: out[i - lo] = f(bits i). */
void orc_encode_range(uint64_t lo, uint64_t hi, uint8_t* out) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t i = (int64_t)lo; i < (int64_t)hi; ++i)
    out[i - (int64_t)lo] = orc_float_to_e4m3(float_of((uint32_t)i));
}

void orc_bf16_range(uint64_t lo, uint64_t hi, uint16_t* out) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t i = (int64_t)lo; i < (int64_t)hi; ++i)
    out[i - (int64_t)lo] = orc_float_to_bf16(float_of((uint32_t)i));
}

void orc_half_range(uint64_t lo, uint64_t hi, uint16_t* out) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t i = (int64_t)lo; i < (int64_t)hi; ++i)
    out[i - (int64_t)lo] = orc_float_to_half(float_of((uint32_t)i));
}
