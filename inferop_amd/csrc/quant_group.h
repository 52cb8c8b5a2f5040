// The quantizer's per-group arithmetic, shared by the quantizer kernels
// (quant.hip) and the GEMM that quantizes its own activations (gemm.hip):
// one 128-element group held by the 16 lanes of a DPP row, 8 elements per
// lane, byte-exact with reference/reference.cpp:65-80.  Compiled by hipcc only.
#pragma once

#include "device_common.h"
#include "quant_math.h"

namespace inferop_hip {
namespace qgroup {

using inferop_qmath::kFastMinAbsmaxBits;
using inferop_qmath::kInv448;

// Per-dtype view of the 8 elements a lane owns, held as raw 32-bit words.
template <int DT>
struct In;

template <>
struct In<kBf16> {
  static constexpr int kWords = 4;
  static constexpr uint32_t kInfKey = 0x7F80u;
  __device__ static float elem(const uint32_t* w, int i) {
    return (i & 1) ? u2f(w[i >> 1] & 0xFFFF0000u) : u2f(w[i >> 1] << 16);
  }
  __device__ static float key_to_float(uint32_t key) { return u2f(key << 16); }
  __device__ static uint32_t key(const uint32_t* w) {
    u16x2 m = __builtin_bit_cast(u16x2, w[0] & 0x7FFF7FFFu);
#pragma unroll
    for (int i = 1; i < kWords; ++i)
      m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[i] & 0x7FFF7FFFu));
    return max((uint32_t)m.x, (uint32_t)m.y);
  }
};

template <>
struct In<kFp16> {
  static constexpr int kWords = 4;
  static constexpr uint32_t kInfKey = 0x7C00u;
  __device__ static float elem(const uint32_t* w, int i) {
    const uint16_t h = (i & 1) ? uint16_t(w[i >> 1] >> 16) : uint16_t(w[i >> 1]);
    return (float)__builtin_bit_cast(_Float16, h);
  }
  __device__ static float key_to_float(uint32_t key) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)key);
  }
  __device__ static uint32_t key(const uint32_t* w) {
    u16x2 m = __builtin_bit_cast(u16x2, w[0] & 0x7FFF7FFFu);
#pragma unroll
    for (int i = 1; i < kWords; ++i)
      m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[i] & 0x7FFF7FFFu));
    return max((uint32_t)m.x, (uint32_t)m.y);
  }
};

template <>
struct In<kFp32> {
  static constexpr int kWords = 8;
  static constexpr uint32_t kInfKey = 0x7F800000u;
  __device__ static float elem(const uint32_t* w, int i) { return u2f(w[i]); }
  __device__ static float key_to_float(uint32_t key) { return u2f(key); }
  __device__ static uint32_t key(const uint32_t* w) {
    uint32_t m = w[0] & 0x7FFFFFFFu;
#pragma unroll
    for (int i = 1; i < kWords; ++i) m = max(m, w[i] & 0x7FFFFFFFu);
    return m;
  }
};

// Magnitude bits of an fp32 value with NaN mapped to 0 (std::max semantics:
// a NaN element never becomes the running maximum).
__device__ __forceinline__ uint32_t mag_nonan(float v) {
  const uint32_t a = f2u(v) & 0x7FFFFFFFu;
  return a > 0x7F800000u ? 0u : a;
}

// Reference-exact code for any x and any scale (slow path).
__device__ __forceinline__ uint32_t slow_code(float x, float s) {
  if (x != x) return ((f2u(x) >> 24) & 0x80u) | 0x7Fu;
  const float qv = x / s;
  if (qv != qv) return 0xFFu;
  return sw_e4m3(qv);
}

// Quantize the 128-element group held by the 16 lanes of one DPP row, each
// lane owning 8 consecutive elements as raw dt words w[]: returns this lane's
// 8 codes (lo = elements 0-3, hi = 4-7) and the group scale.  Every lane of
// the wave must call it (the absmax reduction is a row-wide DPP exchange).
template <int DT>
__device__ __forceinline__ void quant_group_lane(const uint32_t* w, uint32_t& lo, uint32_t& hi,
                                                 float& s) {
  using I = In<DT>;
  uint32_t key = row16_max_u32(I::key(w));
  float amax = I::key_to_float(key);
  s = (key == 0) ? 1.0f : amax * kInv448;
  const bool slow = key >= I::kInfKey || (key != 0 && f2u(amax) < kFastMinAbsmaxBits);
  if (!slow) {
    float v[8];
    if constexpr (DT == kFp32) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = I::elem(w, i) / s;
    } else {
      const float r = 1.0f / s;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = inferop_qmath::div_by_recip(I::elem(w, i), s, r);
    }
    lo = cvt_pk4_e4m3(v[0], v[1], v[2], v[3]);
    hi = cvt_pk4_e4m3(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t k2 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) k2 = max(k2, mag_nonan(I::elem(w, i)));
    k2 = row16_max_u32(k2);
    s = (k2 == 0) ? 1.0f : u2f(k2) * kInv448;
    uint32_t c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = slow_code(I::elem(w, i), s);
    lo = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
    hi = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
  }
}

}  // namespace qgroup
}  // namespace inferop_hip
