// Per-token-group FP8 (E4M3) quantizer and dequantizer for gfx950.
//
// Semantics (byte-exact with reference/reference.cpp:65-80 as compiled for
// x86-64): per group of `group_size` consecutive elements of a row,
//   absmax = max |x| ignoring NaN
//   scale  = absmax == 0 ? 1 : absmax * fl32(1/448)
//   q      = e4m3_rn_sat(x / scale), x / scale correctly rounded.
//
// Fast kernel (group_size == 128, 16-byte aligned input): one 128-element
// group is one 16-lane DPP row, each lane owns 8 consecutive elements (one
// 16-byte load for bf16/fp16, two for fp32) so a wave moves 4 whole groups
// per load instruction, fully coalesced.  absmax is an integer max over the
// magnitude bits (v_pk_max_u16 for 16-bit inputs) followed by a 4-step DPP
// row reduction; no LDS, no barriers.
//
// The quotient: for fp32 input it is the IEEE division.  For bf16 / fp16
// input it is r = 1/scale (IEEE, once per group) then the Markstein
// correction q0 = x*r, e = fma(-q0, scale, x), q = fma(e, r, q0), with the
// sign of x restored (the correction can turn -0 into +0).  The test-suite
// checks every (x, absmax) pair of bf16 and fp16 values the fast path admits:
// q == x/scale bit for bit wherever |x/scale| >= 2^-11, and the E4M3 byte
// equal everywhere.  The E4M3 encode is the hardware
// v_cvt_pk_fp8_f32, proven equal to the reference encoder on that domain by
// inferop_selftest_fp8_codec.
//
// Groups containing Inf/NaN, or with 0 < absmax < 2^-80 (where the quotient
// residual or the scale can be subnormal), take a per-group slow path with the IEEE division and
// the software encoder, and reproduce x86-64 NaN results: a NaN element keeps
// its sign (0x7F / 0xFF), an invalid quotient (0/0, Inf/Inf) is the negative
// default NaN (0xFF).
#include <atomic>
#include <mutex>

#include "device_common.h"
#include "hip_launch.h"
#include "quant_group.h"
#include "quant_math.h"

namespace inferop_hip {
namespace {

using inferop_qmath::kFastMinAbsmaxBits;
using inferop_qmath::kInv448;
using qgroup::In;
using qgroup::mag_nonan;
using qgroup::quant_group_lane;
using qgroup::slow_code;

// NTL / NTS: non-temporal loads / stores (see launch_quant for the choice)
template <int DT, int U, bool NTL = true, bool NTS = true>
__global__ __launch_bounds__(256) void quant_g128_kernel(uint8_t* __restrict__ q,
                                                         float* __restrict__ scales,
                                                         const uint32_t* __restrict__ x,
                                                         int64_t ngroups) {
  using I = In<DT>;
  constexpr int W = I::kWords;
  constexpr int kGroupWords = W * 16;  // 32-bit words per 128-element group
  const int lane = threadIdx.x & 63;
  const int sub = lane & 15;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t g0 = wave * (4 * U) + (lane >> 4);

  uint32_t w[U][W];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t g = g0 + 4 * u;
    if (g < ngroups) {
      const u32x4* src = reinterpret_cast<const u32x4*>(x + g * kGroupWords + sub * W);
#pragma unroll
      for (int v = 0; v < W / 4; ++v) {
        const u32x4 t = NTL ? __builtin_nontemporal_load(src + v) : src[v];
        w[u][4 * v + 0] = t.x;
        w[u][4 * v + 1] = t.y;
        w[u][4 * v + 2] = t.z;
        w[u][4 * v + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) w[u][i] = 0;
    }
  }

#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t g = g0 + 4 * u;
    uint32_t lo, hi;
    float s;
    quant_group_lane<DT>(w[u], lo, hi, s);
    if (g < ngroups) {
      u32x2* dst = reinterpret_cast<u32x2*>(q + g * 128 + sub * 8);
      if (NTS) {
        __builtin_nontemporal_store(u32x2{lo, hi}, dst);
      } else {
        *dst = u32x2{lo, hi};
      }
      if (sub == 0) scales[g] = s;
    }
  }
}

// Any group size, any alignment: one wave per group, grid-stride.
template <int DT>
__device__ __forceinline__ float load_elem(const void* x, int64_t i) {
  if constexpr (DT == kFp32) {
    return reinterpret_cast<const float*>(x)[i];
  } else if constexpr (DT == kBf16) {
    return u2f(uint32_t(reinterpret_cast<const uint16_t*>(x)[i]) << 16);
  } else {
    return (float)reinterpret_cast<const _Float16*>(x)[i];
  }
}

template <int DT>
__global__ __launch_bounds__(256) void quant_generic_kernel(uint8_t* __restrict__ q,
                                                            float* __restrict__ scales,
                                                            const void* __restrict__ x,
                                                            int64_t ngroups, int gs) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); g < ngroups; g += nwaves) {
    const int64_t base = g * gs;
    uint32_t key = 0;
    for (int i = lane; i < gs; i += 64) key = max(key, mag_nonan(load_elem<DT>(x, base + i)));
    key = row16_max_u32(key);
    key = max(max((uint32_t)__builtin_amdgcn_readlane((int)key, 0),
                  (uint32_t)__builtin_amdgcn_readlane((int)key, 16)),
              max((uint32_t)__builtin_amdgcn_readlane((int)key, 32),
                  (uint32_t)__builtin_amdgcn_readlane((int)key, 48)));
    const float s = (key == 0) ? 1.0f : u2f(key) * kInv448;
    for (int i = lane; i < gs; i += 64) q[base + i] = (uint8_t)slow_code(load_elem<DT>(x, base + i), s);
    if (lane == 0) scales[g] = s;
  }
}

// ---- dequantizer: x = dt(e4m3_to_float(q) * scale)  (reference quant.cu:37-46)
// Vector path: 8 elements per lane, so a wave reads 512 contiguous bytes of
// codes and writes its outputs contiguously -- one 16-byte store per lane for
// 16-bit outputs, two for fp32 (4096x7168: bf16 20.9 -> 18.5 us, fp32 44.6 ->
// 31.5 us against 16 elements per lane, whose per-lane 32 / 64 output bytes
// left each store instruction a quarter or half of every cache line).
// NTS: non-temporal stores of 16-bit outputs (see launch_dequant)
template <int DT, bool NTS = false>
__global__ __launch_bounds__(256) void dequant_v8_kernel(void* __restrict__ x,
                                                         const uint8_t* __restrict__ q,
                                                         const float* __restrict__ scales,
                                                         int64_t nvec, int gs) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= nvec) return;
  const u32x2 b = *reinterpret_cast<const u32x2*>(q + t * 8);
  const float s = scales[(t * 8) / gs];
  const uint32_t words[2] = {b.x, b.y};
  float v[8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const f32x2 lo = cvt_pk2_e4m3_f32<false>(words[i]);
    const f32x2 hi = cvt_pk2_e4m3_f32<true>(words[i]);
    v[4 * i + 0] = lo.x * s;
    v[4 * i + 1] = lo.y * s;
    v[4 * i + 2] = hi.x * s;
    v[4 * i + 3] = hi.y * s;
  }
  using T = typename OutT<DT>::T;
  T* dst = reinterpret_cast<T*>(x) + t * 8;
  if constexpr (DT == kFp32) {
    store4<DT>(dst, v[0], v[1], v[2], v[3]);
    store4<DT>(dst + 4, v[4], v[5], v[6], v[7]);
  } else {
    u32x4 buf;  // the 8 outputs, converted as store4 converts them
    store4<DT>(reinterpret_cast<T*>(&buf), v[0], v[1], v[2], v[3]);
    store4<DT>(reinterpret_cast<T*>(&buf) + 4, v[4], v[5], v[6], v[7]);
    if (NTS) {
      __builtin_nontemporal_store(buf, reinterpret_cast<u32x4*>(dst));
    } else {
      *reinterpret_cast<u32x4*>(dst) = buf;
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void dequant_generic_kernel(void* __restrict__ x,
                                                              const uint8_t* __restrict__ q,
                                                              const float* __restrict__ scales,
                                                              int64_t total, int gs) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const float v = inferop::fp8::e4m3_to_float(q[i]) * scales[i / gs];
  store1<DT>(reinterpret_cast<typename OutT<DT>::T*>(x) + i, v);
}

template <int DT>
hipError_t launch_quant(void* q, float* scales, const void* x, int64_t rows, int64_t cols, int gs,
                        hipStream_t st) {
  const int64_t ngroups = rows * (cols / gs);
  const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 8 == 0) && ((uintptr_t)scales % 4 == 0);
  if (gs == 128 && aligned) {
    // two groups per lane for large inputs (4096x7168: 16.1 us vs 18.4 with
    // one; 1024x7168: 5.6 vs 6.2 us); one up to 32768 groups, where the
    // launch has few groups to spread over the GPU (64x7168: 2.5 vs 2.8 us,
    // 512x7168: 3.6 vs 3.9 us)
    if (ngroups <= 32768) {
      const int64_t blocks = (ngroups + 15) / 16;
      hipLaunchKernelGGL((quant_g128_kernel<DT, 1>), dim3((unsigned)blocks), dim3(256), 0, st,
                         (uint8_t*)q, scales, (const uint32_t*)x, ngroups);
    } else {
      constexpr int U = 2;
      const int64_t per_block = 16 * U;
      const int64_t blocks = (ngroups + per_block - 1) / per_block;
      if (blocks > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
      // Cached loads and stores while input and codes together fit the
      // 256 MiB Infinity Cache (4096x7168 bf16: 16.3 -> 16.0 us, 4096x16384:
      // 33.9 -> 33.3 us; fp32 4096x7168 28.1 -> 26.3 us); beyond it
      // non-temporal loads, which keep the input stream from evicting the
      // codes, with cached stores for 16-bit inputs (8192x18432 bf16: 71.9 ->
      // 69.5 us; cached loads there 79.6 us) and non-temporal ones for fp32
      // (cached: 130.5 -> 134.4 us).  Below 64 MiB both stay non-temporal
      // (1024x7168 bf16 with cached ones: 5.8 -> 6.7 us).
      // input bytes per element (kWords words carry 8 elements) plus the code
      const int64_t bytes = rows * cols * (int64_t)(In<DT>::kWords / 2 + 1);
      auto fn = bytes < (int64_t)64 << 20     ? quant_g128_kernel<DT, U, true, true>
                : bytes <= (int64_t)256 << 20 ? quant_g128_kernel<DT, U, false, false>
                                              : quant_g128_kernel<DT, U, true, DT == kFp32>;
      hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(256), 0, st, (uint8_t*)q, scales,
                         (const uint32_t*)x, ngroups);
    }
  } else {
    int64_t blocks = (ngroups + 3) / 4;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL((quant_generic_kernel<DT>), dim3((unsigned)blocks), dim3(256), 0, st,
                       (uint8_t*)q, scales, x, ngroups, gs);
  }
  return hipGetLastError();
}

template <int DT>
hipError_t launch_dequant(void* x, const uint8_t* q, const float* scales, int64_t rows,
                          int64_t cols, int gs, hipStream_t st) {
  const int64_t total = rows * cols;
  const bool vec = (gs % 8 == 0) && ((uintptr_t)q % 8 == 0) && ((uintptr_t)x % 16 == 0) &&
                   total % 8 == 0;
  if (vec) {
    const int64_t nvec = total / 8;
    const int64_t blocks = (nvec + 255) / 256;
    if (blocks > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    // 16-bit outputs: non-temporal stores outside 64..256 MiB of codes and
    // outputs (bf16, A/B on one box: 8192x18432 77.2 -> 72.2 us, 1024x7168
    // 5.7 -> 5.1 us); inside that band, where codes and outputs fit the
    // Infinity Cache, cached stores (8192x7168: 29.5 against 30.2 us).  fp32
    // outputs keep cached stores: a lane's two 16-byte stores cover half
    // lines each, and non-temporal ones took 4096x7168 from 28.5 to 38 us.
    const int64_t bytes = total * (int64_t)(1 + sizeof(typename OutT<DT>::T));
    const bool nts = DT != kFp32 && (bytes < (int64_t)64 << 20 || bytes > (int64_t)256 << 20);
    auto fn = nts ? dequant_v8_kernel<DT, true> : dequant_v8_kernel<DT, false>;
    hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(256), 0, st, x, q, scales, nvec, gs);
  } else {
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((dequant_generic_kernel<DT>), dim3((unsigned)blocks), dim3(256), 0, st, x, q,
                       scales, total, gs);
  }
  return hipGetLastError();
}


// ---- weight block quantizer: one 128 x 128 block of W [N, K] per workgroup ------
// Semantics (the weight recipe of the reference's GEMM tests,
// tests/test_gemm.cpp:28-45): per block, absmax over its rows (ignoring NaN),
// scale = absmax == 0 ? 1 : absmax * fl32(1/448), inv = 1 / scale (IEEE), and
// q = e4m3_rn_sat(w * inv) -- a product with the reciprocal, not a quotient.
// Thread t owns 8 columns (slot t % 16) of rows t / 16 + 16 i.  Blocks
// whose absmax is Inf/NaN or below 2^-80 take the slow path (software encoder,
// x86-64 NaN results, as in the per-token quantizer); elsewhere |w * inv| <=
// 448 and products are never subnormal, so the hardware multiply and encode
// are exact.

// Reference-exact code of w * inv for any w and inv.
__device__ __forceinline__ uint32_t slow_code_mul(float w, float inv) {
  if (w != w) return ((f2u(w) >> 24) & 0x80u) | 0x7Fu;
  const float p = w * inv;
  if (p != p) return 0xFFu;
  return sw_e4m3(p);
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o));
  __syncthreads();  // red[] may still be read by an earlier reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return max(max(red[0], red[1]), max(red[2], red[3]));
}

template <int DT>
__global__ __launch_bounds__(256) void weight_block_quant_kernel(uint8_t* __restrict__ q,
                                                                 float* __restrict__ scales,
                                                                 const void* __restrict__ w,
                                                                 int64_t n, int64_t k) {
  __shared__ uint32_t red[4];
  constexpr int kRows = 8;  // rows per thread
  const int t = threadIdx.x;
  const int c = t & 15;
  const int64_t kg = k >> 7;
  const int64_t g = blockIdx.x, nb = blockIdx.y;
  // columns of thread t: 16-bit inputs 8 consecutive ones (16 bytes, so 16
  // lanes read a row's 256 bytes with one instruction); fp32 inputs two runs
  // of 4, at c * 4 and 64 + c * 4, so each of the two 16-byte loads of a row
  // covers 256 contiguous bytes (rather than half of every 32 bytes)
  const int64_t col = g * 128 + c * (DT == kFp32 ? 4 : 8);
  constexpr int64_t kHiCol = DT == kFp32 ? 64 : 4;  // offset of columns 4..7
  // the block's values stay in registers as loaded (16-bit inputs packed two
  // to a word: half the registers of fp32 copies, so more workgroups per CU)
  constexpr int W = DT == kFp32 ? 8 : 4;
  uint32_t wv[kRows][W];
  auto val = [&](int i, int j) -> float {
    if constexpr (DT == kFp32) {
      return u2f(wv[i][j]);
    } else if constexpr (DT == kBf16) {
      return u2f((j & 1) ? (wv[i][j >> 1] & 0xFFFF0000u) : (wv[i][j >> 1] << 16));
    } else {
      return (float)__builtin_bit_cast(
          _Float16, (uint16_t)((j & 1) ? (wv[i][j >> 1] >> 16) : (wv[i][j >> 1] & 0xFFFFu)));
    }
  };
  // the codes of the thread's columns 0..3 (lo) and 4..7 (hi) of a row.  The
  // weight is read once and its codes written once: both go non-temporal
  // (7168x16384 fp32 110 -> 99 us, 36864x7168 bf16 142 -> 135 us, fp16 145 ->
  // 136 us).
  auto store_codes = [&](uint8_t* dst, uint32_t lo, uint32_t hi) {
    if constexpr (DT == kFp32) {
      __builtin_nontemporal_store(lo, reinterpret_cast<uint32_t*>(dst));
      __builtin_nontemporal_store(hi, reinterpret_cast<uint32_t*>(dst + kHiCol));
    } else {
      __builtin_nontemporal_store(u32x2{lo, hi}, reinterpret_cast<u32x2*>(dst));
    }
  };
  uint32_t key = 0;
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const int64_t row = nb * 128 + (t >> 4) + 16 * i;
    if (row < n) {
      const int64_t e = row * k + col;
      if constexpr (DT == kFp32) {
        const float* p = reinterpret_cast<const float*>(w) + e;
        const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + kHiCol));
        wv[i][0] = a.x, wv[i][1] = a.y, wv[i][2] = a.z, wv[i][3] = a.w;
        wv[i][4] = b.x, wv[i][5] = b.y, wv[i][6] = b.z, wv[i][7] = b.w;
      } else {
        const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(w) + e));
        wv[i][0] = a.x, wv[i][1] = a.y, wv[i][2] = a.z, wv[i][3] = a.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < W; ++j) wv[i][j] = 0u;
    }
    if constexpr (DT == kBf16) {
      // |value| bits straight from the packed words (no fp32 copies kept)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        key = max(key, max((wv[i][j] << 16) & 0x7FFFFFFFu, wv[i][j] & 0x7FFF0000u));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) key = max(key, f2u(val(i, j)) & 0x7FFFFFFFu);
    }
  }
  key = block_max_u32(key, red);
  const bool slow = key >= 0x7F800000u || (key != 0 && key < kFastMinAbsmaxBits);
  float s;
  if (!slow) {
    s = (key == 0) ? 1.0f : u2f(key) * kInv448;
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int64_t row = nb * 128 + (t >> 4) + 16 * i;
      if (row < n) {
        const uint32_t lo = cvt_pk4_e4m3(val(i, 0) * inv, val(i, 1) * inv, val(i, 2) * inv, val(i, 3) * inv);
        const uint32_t hi = cvt_pk4_e4m3(val(i, 4) * inv, val(i, 5) * inv, val(i, 6) * inv, val(i, 7) * inv);
        store_codes(q + row * k + col, lo, hi);
      }
    }
  } else {
    // rare blocks (Inf/NaN or a tiny absmax): the rows are read again from
    // memory one at a time, so this path holds no block copy in registers
    auto row_vals = [&](int i, float* x) {
      const int64_t row = nb * 128 + (t >> 4) + 16 * i;
      if (row >= n) {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = 0.0f;
        return;
      }
      const int64_t e = row * k + col;
      if constexpr (DT == kFp32) {
        const float* p = reinterpret_cast<const float*>(w) + e;
        const u32x4 a = *reinterpret_cast<const u32x4*>(p);
        const u32x4 b = *reinterpret_cast<const u32x4*>(p + kHiCol);
        const uint32_t r[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = u2f(r[j]);
      } else {
        const u32x4 a = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(w) + e);
        const uint32_t r[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (DT == kBf16) {
            x[2 * j] = u2f(r[j] << 16);
            x[2 * j + 1] = u2f(r[j] & 0xFFFF0000u);
          } else {
            x[2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r[j] & 0xFFFFu));
            x[2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r[j] >> 16));
          }
        }
      }
    };
    uint32_t k2 = 0;
#pragma unroll 1
    for (int i = 0; i < kRows; ++i) {
      float x[8];
      row_vals(i, x);
#pragma unroll
      for (int j = 0; j < 8; ++j) k2 = max(k2, mag_nonan(x[j]));
    }
    k2 = block_max_u32(k2, red);
    s = (k2 == 0) ? 1.0f : u2f(k2) * kInv448;
    const float inv = 1.0f / s;
#pragma unroll 1
    for (int i = 0; i < kRows; ++i) {
      const int64_t row = nb * 128 + (t >> 4) + 16 * i;
      if (row < n) {
        float x[8];
        row_vals(i, x);
        uint32_t cd[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) cd[j] = slow_code_mul(x[j], inv);
        store_codes(q + row * k + col, cd[0] | (cd[1] << 8) | (cd[2] << 16) | (cd[3] << 24),
                    cd[4] | (cd[5] << 8) | (cd[6] << 16) | (cd[7] << 24));
      }
    }
  }
  if (t == 0) scales[nb * kg + g] = s;
}

template <int DT>
hipError_t launch_weight_quant(uint8_t* q, float* scales, const void* w, int64_t n, int64_t k,
                               hipStream_t st) {
  const int64_t kg = k / 128, nb = (n + 127) / 128;
  if (kg > 0x7FFFFFFF || nb > 65535) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((weight_block_quant_kernel<DT>), dim3((unsigned)kg, (unsigned)nb), dim3(256), 0,
                     st, q, scales, w, n, k);
  return hipGetLastError();
}


// ---- fused producers: the layer output is quantized without a dt round trip ----
// Each computes the producer in fp32, rounds the value to the storage type dt
// exactly where the unfused path stores it (round to nearest even: the
// hardware conversions (__bf16) / (_Float16), i.e. __float2bfloat16 /
// __float2half of the reference kernels), and quantizes that value with the
// per-token-group quantizer above -- bytes and scales are those of
// quant_fp8_per_token_group applied to the stored producer output.

// 8 fp32 values rounded to dt, packed as the raw words quant_group_lane reads.
template <int DT>
__device__ __forceinline__ void pack_dt8(const float* v, uint32_t* w) {
  if constexpr (DT == kFp32) {
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = f2u(v[i]);
  } else if constexpr (DT == kBf16) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = uint32_t(__builtin_bit_cast(uint16_t, (__bf16)v[2 * i])) |
             (uint32_t(__builtin_bit_cast(uint16_t, (__bf16)v[2 * i + 1])) << 16);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = uint32_t(__builtin_bit_cast(uint16_t, to_fp16(v[2 * i]))) |
             (uint32_t(__builtin_bit_cast(uint16_t, to_fp16(v[2 * i + 1]))) << 16);
  }
}

// 8 consecutive dt elements at p (16-byte aligned for 16-bit types, 32 for fp32).
template <int DT, bool NT = false>
__device__ __forceinline__ void load_dt8(const void* p, float* v) {
  auto ld = [](const u32x4* a) { return NT ? __builtin_nontemporal_load(a) : *a; };
  if constexpr (DT == kFp32) {
    const u32x4* q = reinterpret_cast<const u32x4*>(p);
    const u32x4 a = ld(q), b = ld(q + 1);
    v[0] = u2f(a.x), v[1] = u2f(a.y), v[2] = u2f(a.z), v[3] = u2f(a.w);
    v[4] = u2f(b.x), v[5] = u2f(b.y), v[6] = u2f(b.z), v[7] = u2f(b.w);
  } else {
    const u32x4 a = ld(reinterpret_cast<const u32x4*>(p));
    const uint32_t ws[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == kBf16) {
        v[2 * i] = u2f(ws[i] << 16);
        v[2 * i + 1] = u2f(ws[i] & 0xFFFF0000u);
      } else {
        v[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)ws[i]);
        v[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(ws[i] >> 16));
      }
    }
  }
}

// SiLU(g) * u with the reference's fp32 operation order
// (reference/reference.cpp:60-61: (g / (1 + exp(-g))) * u).  exp(-g) is
// evaluated in double precision and rounded once to fp32, which gives the
// correctly rounded fp32 exponential except where the double result lies
// within 2^-29 relative of an fp32 rounding midpoint.
__device__ __forceinline__ float silu_of(float g) {
  const float e = (float)::exp(-(double)g);
  return g / (1.0f + e);
}
__device__ __forceinline__ float silu_mul(float g, float u) { return silu_of(g) * u; }

// For 16-bit gates, g / (1 + exp(-g)) depends only on the gate's 16 bits: a
// table of the fp32 value for each of the 65536 patterns (built on the device
// by silu_of, so the entries are bit for bit what the arithmetic above
// gives), indexed by the bits, leaves one gather and the reference's final
// multiply per element (bf16 4096x18432: 146 -> 111 us on one box).  The bf16
// gates of a layer touch a few thousand entries, which stay in the L1 cache;
// fp16 gates, with 10-bit mantissas, spread over about 8 times as many, and
// gathers from the full fp16 table cost more than the arithmetic (181 us
// against about 146 us), so large calls gather from a slice of each table
// held in LDS (below).  One set of tables per GPU (static device memory,
// held until the process ends), built by silu_table_build_kernel at the
// first bf16 or fp16 call on the device (see launch_silu_mul_quant); a
// launch that finds no table evaluates the arithmetic instead, and both give
// the same bits.
__device__ float silu_table_bf16[65536];
__device__ float silu_table_f16[65536];

__global__ __launch_bounds__(256) void silu_table_build_kernel() {
  const uint32_t b = blockIdx.x * 256 + threadIdx.x;
  silu_table_bf16[b] = silu_of(u2f(b << 16));
  silu_table_f16[b] = silu_of((float)__builtin_bit_cast(_Float16, (uint16_t)b));
}

// Most of the table is one of three exact rules.  For a bf16 gate g with
// exponent field E (bits 14..7):
//   E <  102 (|g| < 2^-25): exp(-g) rounds to 1, so the value is g / 2 = g * 0.5f;
//   E >= 134 (|g| >= 128), finite: g > 0 gives exp(-g) < 2^-24, 1 + e rounds
//     to 1 and the value is g; g < 0 gives exp(-g) = +Inf and the value -0;
//   E == 255 with g > 0 (+Inf, NaN): the value is g (NaN keeps its sign);
//   E == 255 with g < 0 (-Inf, NaN): read from the full table.
// Only E in [102, 134) for both signs needs the table: 2 x 32 x 128 entries,
// 32 KB, which a workgroup copies into LDS once and then gathers from LDS
// instead of the global table's L1/L2 gathers (the test-suite checks the
// rules against the oracle's SiLU over every bf16 pattern).
constexpr uint32_t kSiluLdsLoExp = 102;
constexpr int kSiluLdsEntries = 2 * 32 * 128;

// Slice of the full table for LDS entry i: (sign << 12) | ((E - 102) << 7) | m
// sits at bf16 bits (sign << 15) | ((102 << 7) + (i & 4095)).
template <int NT>
__device__ __forceinline__ void silu_lds_fill(float* tab) {
  const u32x4* src = reinterpret_cast<const u32x4*>(silu_table_bf16);
  u32x4* dst = reinterpret_cast<u32x4*>(tab);
#pragma unroll
  for (int j = 0; j < kSiluLdsEntries / 4 / NT; ++j) {
    const int v = j * NT + (int)threadIdx.x;  // 16-byte chunk of the slice
    const int i = v * 4;
    dst[v] = src[(((uint32_t)i >> 12) << 13) + ((kSiluLdsLoExp << 7) + (i & 4095)) / 4];
  }
}

// silu(g) for the bf16 gate whose bits are the upper half of gbits.
__device__ __forceinline__ float silu_bf16_lds(const float* tab, uint32_t gbits) {
  const uint32_t b = gbits >> 16;
  const uint32_t e = (b >> 7) & 0xFFu;
  const uint32_t rel = e - kSiluLdsLoExp;  // wraps for e < 102
  const float t = tab[((b >> 15) << 12) | ((rel & 31u) << 7) | (b & 0x7Fu)];
  const float g = u2f(gbits);
  const float rule = e < kSiluLdsLoExp ? g * 0.5f : ((b >> 15) ? -0.0f : g);
  return rel < 32u ? t : rule;
}

// fp16 gates: the slice of silu_table_f16 for exponent fields [11, 17)
// (2^-4 <= |g| < 4) of both signs, 2 x 6 x 1024 entries, 48 KB (three
// workgroups per CU), holds all but about 5% of normally distributed gates;
// the rest (and Inf / NaN) gather from the full table.  LDS entry
// i = sign * 6144 + (E - 11) * 1024 + mantissa.  Measured on 4096x18432
// (graph over > 1 GiB of inputs): the double exponential pair this replaced
// 119-122 us; slices of 8 exponents (64 KB, two workgroups per CU) 96 us,
// 6 exponents 92 us, 5 (four per CU) 93-96 us, 4 exponents 113 us.
constexpr uint32_t kSiluF16LoExp = 11;
constexpr int kSiluF16Exps = 6;
constexpr int kSiluF16LdsEntries = 2 * kSiluF16Exps * 1024;

template <int NT>
__device__ __forceinline__ void silu_f16_lds_fill(float* tab) {
  static_assert(kSiluF16LdsEntries % (4 * NT) == 0, "whole 16-byte chunks per thread");
  const u32x4* src = reinterpret_cast<const u32x4*>(silu_table_f16);
  u32x4* dst = reinterpret_cast<u32x4*>(tab);
#pragma unroll
  for (int j = 0; j < kSiluF16LdsEntries / 4 / NT; ++j) {
    const int v = j * NT + (int)threadIdx.x;  // 16-byte chunk of the slice
    const uint32_t i = (uint32_t)v * 4;
    const uint32_t sign = i / (kSiluF16Exps * 1024), e = kSiluF16LoExp + (i >> 10) % kSiluF16Exps;
    dst[v] = src[((sign << 15) | (e << 10) | (i & 1023u)) / 4];
  }
}

// silu(g) for the fp16 gate g (exactly representable in fp16).
__device__ __forceinline__ float silu_f16_lds(const float* tab, float g) {
  const uint32_t b = __builtin_bit_cast(uint16_t, (_Float16)g);
  const uint32_t rel = ((b >> 10) & 31u) - kSiluF16LoExp;  // wraps below the slice
  return rel < (uint32_t)kSiluF16Exps
             ? tab[(b >> 15) * (kSiluF16Exps * 1024) + (rel << 10) + (b & 1023u)]
             : silu_table_f16[b];
}

// gate_up: [tokens, 2d] dt (bf16 or fp16) -> q [tokens, d] E4M3, scales
// [tokens, d/128], with a slice of the SiLU table in LDS (bf16: 32 KB; fp16:
// 48 KB).  Lane layout as silu_mul_quant_kernel (16
// lanes per 128-output group, 4 groups per wave and step, U steps issued
// together); NT-thread workgroups stride over the groups so each copies the
// tables once, and large workgroups let more waves share one copy.
template <int DT, int U, int NT>
__global__ __launch_bounds__(NT) void silu_mul_quant_lds_kernel(uint8_t* __restrict__ q,
                                                                 float* __restrict__ scales,
                                                                 const uint16_t* __restrict__ gate_up,
                                                                 uint32_t d, uint32_t gpr,
                                                                 uint32_t ngroups) {
  static_assert(DT == kBf16 || DT == kFp16, "16-bit gates only");
  constexpr int kBytes = (DT == kBf16 ? kSiluLdsEntries : kSiluF16LdsEntries) * 4;
  __shared__ __align__(16) uint8_t lds[kBytes];
  float* tab = reinterpret_cast<float*>(lds);
  if constexpr (DT == kBf16) {
    silu_lds_fill<NT>(tab);
  } else {
    silu_f16_lds_fill<NT>(tab);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int sub = lane & 15;
  const uint32_t wave = threadIdx.x >> 6;
  for (uint32_t step = blockIdx.x;; step += gridDim.x) {
    const uint64_t base = ((uint64_t)step * (NT / 64) + wave) * (4 * U);
    if (base >= ngroups) break;  // uniform over the wave
    float gv[U][8], uv[U][8];
    uint32_t t[U], gc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = (uint32_t)base + 4 * u + (lane >> 4);
      t[u] = g / gpr;
      gc[u] = g - t[u] * gpr;
      if (g < ngroups) {
        const uint16_t* row = gate_up + (uint64_t)t[u] * 2 * d + gc[u] * 128 + sub * 8;
        load_dt8<DT, true>(row, gv[u]);
        load_dt8<DT, true>(row + d, uv[u]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) gv[u][i] = uv[u][i] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = (uint32_t)base + 4 * u + (lane >> 4);
      float y[8];
      if constexpr (DT == kBf16) {
        bool special = false;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          y[i] = silu_bf16_lds(tab, f2u(gv[u][i]));
          special |= (f2u(gv[u][i]) >> 23) == 0x1FFu;
        }
        if (special) {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if ((f2u(gv[u][i]) >> 23) == 0x1FFu) y[i] = silu_table_bf16[f2u(gv[u][i]) >> 16];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = silu_f16_lds(tab, gv[u][i]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] *= uv[u][i];
      uint32_t w[In<DT>::kWords];
      pack_dt8<DT>(y, w);
      uint32_t lo, hi;
      float s;
      quant_group_lane<DT>(w, lo, hi, s);
      if (g < ngroups) {
        __builtin_nontemporal_store(
            u32x2{lo, hi},
            reinterpret_cast<u32x2*>(q + (uint64_t)t[u] * d + gc[u] * 128 + sub * 8));
        if (sub == 0) scales[g] = s;
      }
    }
  }
}


// gate_up: [tokens, 2d] dt -> q [tokens, d] E4M3, scales [tokens, d/128].
// Lane layout as quant_g128_kernel: 16 lanes per 128-output group, a wave
// covering 4 groups per step and U steps, whose gate and up loads are all
// issued before the first is used (streamed once: non-temporal loads and
// stores).
template <int DT, int U>
__global__ __launch_bounds__(256) void silu_mul_quant_kernel(uint8_t* __restrict__ q,
                                                             float* __restrict__ scales,
                                                             const void* __restrict__ gate_up,
                                                             int64_t d, int64_t ngroups,
                                                             int use_table) {
  constexpr int EB = DT == kFp32 ? 4 : 2;
  const int lane = threadIdx.x & 63;
  const int sub = lane & 15;
  const int64_t g0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * (4 * U) + (lane >> 4);
  const int64_t gpr = d >> 7;
  float gv[U][8], uv[U][8];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t g = g0 + 4 * u;
    if (g < ngroups) {
      const int64_t t = g / gpr, gc = g - t * gpr;
      const uint8_t* row = reinterpret_cast<const uint8_t*>(gate_up) + t * 2 * d * EB;
      load_dt8<DT, true>(row + (gc * 128 + sub * 8) * EB, gv[u]);
      load_dt8<DT, true>(row + (d + gc * 128 + sub * 8) * EB, uv[u]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) gv[u][i] = uv[u][i] = 0.0f;
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t g = g0 + 4 * u;
    float y[8];
    if (DT == kBf16 && use_table) {
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = silu_table_bf16[f2u(gv[u][i]) >> 16] * uv[u][i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = silu_mul(gv[u][i], uv[u][i]);
    }
    uint32_t w[In<DT>::kWords];
    pack_dt8<DT>(y, w);
    uint32_t lo, hi;
    float s;
    quant_group_lane<DT>(w, lo, hi, s);
    if (g < ngroups) {
      const int64_t t = g / gpr, gc = g - t * gpr;
      __builtin_nontemporal_store(u32x2{lo, hi},
                                  reinterpret_cast<u32x2*>(q + t * d + gc * 128 + sub * 8));
      if (sub == 0) scales[g] = s;
    }
  }
}

// One workgroup per row: residual = dt(residual + x) in place, then
// out = dt((residual * inv_rms) * weight) quantized per 128-column group
// (reference/reference.cpp:23-35 for the arithmetic; the sum of squares is a
// tree over the stored residual values, the reference's is left to right).
template <int DT>
__global__ __launch_bounds__(256) void add_rmsnorm_quant_kernel(
    void* __restrict__ residual, uint8_t* __restrict__ q, float* __restrict__ scales,
    const void* __restrict__ x, const void* __restrict__ weight, int64_t cols, float eps) {
  constexpr int EB = DT == kFp32 ? 4 : 2;
  __shared__ float red[4];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  uint8_t* res = reinterpret_cast<uint8_t*>(residual) + row * cols * EB;
  const uint8_t* xr = reinterpret_cast<const uint8_t*>(x) + row * cols * EB;
  // pass 1 stores residual = dt(residual + x) and sums the squares of the
  // stored values; the first kKeep column blocks (cols <= 8192) keep those
  // values in registers for pass 2 (as the stored dt words: half the
  // registers for 16-bit types), longer rows read the rest back
  constexpr int kKeep = 4;
  uint32_t keep[kKeep][In<DT>::kWords];
  float ss = 0.0f;
  auto pass1 = [&](int64_t c, uint32_t* kept) {
    float rv[8], xv[8];
    load_dt8<DT>(res + c * EB, rv);
    load_dt8<DT>(xr + c * EB, xv);
#pragma unroll
    for (int i = 0; i < 8; ++i) rv[i] = rv[i] + xv[i];
    uint32_t w[In<DT>::kWords];
    pack_dt8<DT>(rv, w);
    if constexpr (DT == kFp32) {
      *reinterpret_cast<u32x4*>(res + c * EB) = u32x4{w[0], w[1], w[2], w[3]};
      *reinterpret_cast<u32x4*>(res + c * EB + 16) = u32x4{w[4], w[5], w[6], w[7]};
    } else {
      *reinterpret_cast<u32x4*>(res + c * EB) = u32x4{w[0], w[1], w[2], w[3]};
    }
    float stored[8];
    load_dt8<DT>(w, stored);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += stored[i] * stored[i];
    if (kept) {
#pragma unroll
      for (int i = 0; i < In<DT>::kWords; ++i) kept[i] = w[i];
    }
  };
#pragma unroll
  for (int it = 0; it < kKeep; ++it) {
    const int64_t c = (int64_t)t * 8 + it * 2048;
    if (c < cols) pass1(c, keep[it]);
  }
  for (int64_t c = (int64_t)t * 8 + kKeep * 2048; c < cols; c += 2048) pass1(c, nullptr);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)cols + eps);
  const int64_t gpr = cols >> 7;
  const uint8_t* wt = reinterpret_cast<const uint8_t*>(weight);
  // pass 2: out = dt((residual * inv) * weight), quantized per 128 columns;
  // kept values come from registers, the rest from this thread's own stores
  auto pass2 = [&](int64_t c0, const uint32_t* kept) {
    const int64_t c = c0 + (int64_t)t * 8;
    const bool live = c < cols;  // whole 16-lane groups, since cols % 128 == 0
    float y[8];
    if (live) {
      float rv[8], wv[8];
      if (kept) {
        load_dt8<DT>(kept, rv);
      } else {
        load_dt8<DT>(res + c * EB, rv);
      }
      load_dt8<DT>(wt + c * EB, wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = rv[i] * inv * wv[i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = 0.0f;
    }
    uint32_t w[In<DT>::kWords];
    pack_dt8<DT>(y, w);
    uint32_t lo, hi;
    float s;
    quant_group_lane<DT>(w, lo, hi, s);
    if (live) {
      *reinterpret_cast<u32x2*>(q + row * cols + c) = u32x2{lo, hi};
      if ((t & 15) == 0) scales[row * gpr + (c >> 7)] = s;
    }
  };
#pragma unroll
  for (int it = 0; it < kKeep; ++it)
    if (it * 2048 < cols) pass2(it * 2048, keep[it]);
  for (int64_t c0 = kKeep * 2048; c0 < cols; c0 += 2048) pass2(c0, nullptr);
}

// The bf16 SiLU table of the current device, built at the first bf16 call on
// the device: the build kernel runs on a library stream that is never
// captured and the host waits for it (once per device), so every later
// launch, on any stream, finds the table complete.  When the first call is
// being captured the wait runs in relaxed capture mode, as the split-K
// workspace set-up does.  Returns false (compute instead) if the build
// failed.
std::once_flag g_silu_table_once[64];
bool g_silu_table_ok[64];
hipStream_t g_silu_table_stream[64];

bool silu_table(hipStream_t caller) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  std::call_once(g_silu_table_once[dev], [&] {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(caller, &cs) != hipSuccess) return;
    const bool capturing = cs != hipStreamCaptureStatusNone;
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    if (capturing && hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return;
    hipError_t e = hipSuccess;
    if (!g_silu_table_stream[dev])
      e = hipStreamCreateWithFlags(&g_silu_table_stream[dev], hipStreamNonBlocking);
    if (e == hipSuccess) {
      hipLaunchKernelGGL(silu_table_build_kernel, dim3(256), dim3(256), 0,
                         g_silu_table_stream[dev]);
      e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(g_silu_table_stream[dev]);
    if (capturing) (void)hipThreadExchangeStreamCaptureMode(&mode);
    g_silu_table_ok[dev] = e == hipSuccess;
  });
  return g_silu_table_ok[dev];
}

// Compute units of the current device (cached per device ordinal).
hipError_t silu_device_cus(int* cus) {
  static std::atomic<int> cached[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev >= 0 && dev < 64 && cached[dev].load(std::memory_order_relaxed) > 0) {
    *cus = cached[dev].load(std::memory_order_relaxed);
    return hipSuccess;
  }
  int v = 0;
  e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  if (v <= 0) return hipErrorInvalidDevice;
  if (dev >= 0 && dev < 64) cached[dev].store(v, std::memory_order_relaxed);
  *cus = v;
  return hipSuccess;
}

// Workgroups per CU of the LDS-table SiLU kernel: four 512-thread
// workgroups (32 KB of LDS each) hold 32 waves per CU at 58 VGPRs.  Measured
// on 4096x18432 bf16 (graph of launches over 1.2 GB of inputs): 4 x 256
// threads 100 us, 8 x 256 (5 resident) 92 us, 2 x 1024 96 us, 4 x 512 84-87
// us; four steps in flight per wave (94 VGPRs, 5 waves per SIMD) 100 us.
constexpr int kSiluLdsWgPerCu = 4;

// The LDS-table kernels take the group count and d as 32-bit values and form
// column offsets (group * 128) in 32 bits: they run only for ngroups < 2^32
// and d < 2^31; anything larger takes the 64-bit kernel below them.
template <int DT>
hipError_t launch_silu_mul_quant(uint8_t* q, float* scales, const void* gate_up, int64_t tokens,
                                 int64_t d, hipStream_t st) {
  const int use_table = DT == kBf16 && silu_table(st) ? 1 : 0;
  const int64_t ngroups = tokens * (d / 128);
  if constexpr (DT == kFp16) {
    if (silu_table(st)) {
      // 48 KB of LDS per workgroup: three 512-thread workgroups per CU
      constexpr int UL = 2, NT = 512, kWgPerCu = 3;
      constexpr int kStep = NT / 16 * UL;
      int cus = 0;
      if (hipError_t e = silu_device_cus(&cus); e != hipSuccess) return e;
      if (ngroups >= (int64_t)kStep * cus && ngroups <= 0xFFFFFFFFll && d <= 0x7FFFFFFF) {
        const int64_t steps = (ngroups + kStep - 1) / kStep;
        const int64_t blocks = steps < (int64_t)cus * kWgPerCu ? steps : (int64_t)cus * kWgPerCu;
        hipLaunchKernelGGL((silu_mul_quant_lds_kernel<kFp16, UL, NT>), dim3((unsigned)blocks),
                           dim3(NT), 0, st, q, scales, static_cast<const uint16_t*>(gate_up),
                           (uint32_t)d, (uint32_t)(d / 128), (uint32_t)ngroups);
        return hipGetLastError();
      }
    }
  }
  if (DT == kBf16 && use_table) {
    // the LDS slice pays for its 32 KB copy once every CU has a full step
    constexpr int UL = 2, NT = 512;
    constexpr int kStep = NT / 16 * UL;  // groups per workgroup step
    int cus = 0;
    if (hipError_t e = silu_device_cus(&cus); e != hipSuccess) return e;
    if (ngroups >= (int64_t)kStep * cus && ngroups <= 0xFFFFFFFFll && d <= 0x7FFFFFFF) {
      const int64_t steps = (ngroups + kStep - 1) / kStep;
      const int64_t blocks = steps < (int64_t)cus * kSiluLdsWgPerCu ? steps
                                                                     : (int64_t)cus * kSiluLdsWgPerCu;
      hipLaunchKernelGGL((silu_mul_quant_lds_kernel<kBf16, UL, NT>), dim3((unsigned)blocks), dim3(NT), 0, st,
                         q, scales, static_cast<const uint16_t*>(gate_up), (uint32_t)d,
                         (uint32_t)(d / 128), (uint32_t)ngroups);
      return hipGetLastError();
    }
  }
  // one step per wave: two or four in flight were no faster (4096x18432 bf16
  // 109 / 112 / 107 us), the table gathers and the arithmetic set the pace
  constexpr int U = 1;
  const int64_t blocks = (ngroups + 16 * U - 1) / (16 * U);
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((silu_mul_quant_kernel<DT, U>), dim3((unsigned)blocks), dim3(256), 0, st, q,
                     scales, gate_up, d, ngroups, use_table);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_add_rmsnorm_quant(void* residual, uint8_t* q, float* scales, const void* x,
                                    const void* weight, int64_t rows, int64_t cols, float eps,
                                    hipStream_t st) {
  if (rows > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((add_rmsnorm_quant_kernel<DT>), dim3((unsigned)rows), dim3(256), 0, st,
                     residual, q, scales, x, weight, cols, eps);
  return hipGetLastError();
}

}  // namespace
}  // namespace inferop_hip

using namespace inferop_hip;

extern "C" int inferop_hip_quant_fp8_group(void* q, float* scales, const void* x, int32_t dt,
                                           int64_t rows, int64_t cols, int32_t group_size,
                                           void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dt) {
    case kFp32: return launch_quant<kFp32>(q, scales, x, rows, cols, group_size, st);
    case kFp16: return launch_quant<kFp16>(q, scales, x, rows, cols, group_size, st);
    case kBf16: return launch_quant<kBf16>(q, scales, x, rows, cols, group_size, st);
    default: return hipErrorInvalidValue;
  }
}

extern "C" int inferop_hip_dequant_fp8_group(void* x, int32_t dt, const uint8_t* q,
                                             const float* scales, int64_t rows, int64_t cols,
                                             int32_t group_size, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dt) {
    case kFp32: return launch_dequant<kFp32>(x, q, scales, rows, cols, group_size, st);
    case kFp16: return launch_dequant<kFp16>(x, q, scales, rows, cols, group_size, st);
    case kBf16: return launch_dequant<kBf16>(x, q, scales, rows, cols, group_size, st);
    default: return hipErrorInvalidValue;
  }
}

extern "C" int inferop_hip_weight_block_quant(uint8_t* q, float* scales, const void* w, int32_t dt,
                                              int64_t n, int64_t k, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the kernel loads 16 bytes and stores 8 bytes per row segment
  if ((uintptr_t)w % 16 != 0 || (uintptr_t)q % 8 != 0 || (uintptr_t)scales % 4 != 0)
    return hipErrorInvalidValue;
  switch (dt) {
    case kFp32: return launch_weight_quant<kFp32>(q, scales, w, n, k, st);
    case kFp16: return launch_weight_quant<kFp16>(q, scales, w, n, k, st);
    case kBf16: return launch_weight_quant<kBf16>(q, scales, w, n, k, st);
    default: return hipErrorInvalidValue;
  }
}

extern "C" int inferop_hip_silu_mul_quant(uint8_t* q, float* scales, const void* gate_up,
                                          int32_t dt, int64_t tokens, int64_t d, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dt) {
    case kFp32: return launch_silu_mul_quant<kFp32>(q, scales, gate_up, tokens, d, st);
    case kFp16: return launch_silu_mul_quant<kFp16>(q, scales, gate_up, tokens, d, st);
    case kBf16: return launch_silu_mul_quant<kBf16>(q, scales, gate_up, tokens, d, st);
    default: return hipErrorInvalidValue;
  }
}

extern "C" int inferop_hip_add_rmsnorm_quant(void* residual, uint8_t* q, float* scales,
                                             const void* x, const void* weight, int32_t dt,
                                             int64_t rows, int64_t cols, float eps, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dt) {
    case kFp32:
      return launch_add_rmsnorm_quant<kFp32>(residual, q, scales, x, weight, rows, cols, eps, st);
    case kFp16:
      return launch_add_rmsnorm_quant<kFp16>(residual, q, scales, x, weight, rows, cols, eps, st);
    case kBf16:
      return launch_add_rmsnorm_quant<kBf16>(residual, q, scales, x, weight, rows, cols, eps, st);
    default: return hipErrorInvalidValue;
  }
}
