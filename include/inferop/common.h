// inferop (MI355X build) : shared types and host-only 16-bit conversions.
//
// Drop-in for the reference header include/inferop/common.h: the same names,
// the same enum values and the same conversion semantics, so code written
// against the reference compiles and produces the same bytes.  Nothing here
// includes HIP: the C++ front end and the CPU tests build with plain g++.
//
// Reference interface replaced: include/inferop/common.h:13-101.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

namespace inferop {

// ABI tag passed by value through ops.h (common.h:13 in the reference).
enum class dtype : int32_t { fp32 = 0, fp16 = 1, bf16 = 2, fp8_e4m3 = 3 };

inline const char* dtype_name(dtype d) {
  switch (d) {
    case dtype::fp32: return "fp32";
    case dtype::fp16: return "fp16";
    case dtype::bf16: return "bf16";
    case dtype::fp8_e4m3: return "fp8_e4m3";
  }
  return "unknown";
}

inline int dtype_bytes(dtype d) {
  switch (d) {
    case dtype::fp32: return 4;
    case dtype::fp16:
    case dtype::bf16: return 2;
    case dtype::fp8_e4m3: return 1;
  }
  return 0;
}

namespace bitcast {
inline float u32_to_f32(uint32_t w) {
  float f;
  std::memcpy(&f, &w, 4);
  return f;
}
inline uint32_t f32_to_u32(float f) {
  uint32_t w;
  std::memcpy(&w, &f, 4);
  return w;
}
}  // namespace bitcast

// Host conversions that define the wire format of 16-bit tensors.
//
// bf16: round-to-nearest-even on the raw bits, with no NaN special case (a
// NaN whose low half rounds up can carry into the sign bit), exactly as the
// reference's float_to_bf16_rn (common.h:57-61).
//
// fp16: round-to-nearest-even with two deliberate departures from IEEE that
// the reference's float_to_half_rn has (common.h:80-101) and that this header
// keeps so packed test inputs are byte-identical:
//   * every finite |f| > 65504 becomes Inf (IEEE would round (65504, 65520)
//     down to 65504);
//   * every |f| < 2^-24 becomes signed zero (IEEE would round (2^-25, 2^-24)
//     up to the smallest subnormal).
// NaN becomes 0x7E00 whatever its sign or payload.
namespace host_convert {

inline float bf16_to_float(uint16_t v) { return bitcast::u32_to_f32(uint32_t(v) << 16); }

inline uint16_t float_to_bf16_rn(float f) {
  const uint32_t w = bitcast::f32_to_u32(f);
  const uint32_t bias = 0x7FFFu + ((w >> 16) & 1u);
  return uint16_t((w + bias) >> 16);
}

inline float half_to_float(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  const uint32_t m = h & 0x3FFu;
  if (e == 0x1Fu) {
    if (m) return std::nanf("");
    return bitcast::u32_to_f32(sign | 0x7F800000u);
  }
  if (e == 0) {
    // subnormal or zero: m * 2^-24 is exact in fp32.
    const float mag = float(m) * 5.9604644775390625e-8f;
    return sign ? -mag : mag;
  }
  return bitcast::u32_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

inline uint16_t float_to_half_rn(float f) {
  const uint32_t w = bitcast::f32_to_u32(f);
  const uint16_t sign = uint16_t((w >> 16) & 0x8000u);
  const uint32_t a = w & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return 0x7E00u;                // NaN
  if (a > 0x477FE000u) return uint16_t(sign | 0x7C00u);  // > 65504 (incl. Inf)
  if (a < 0x33800000u) return sign;                   // < 2^-24
  if (a < 0x38800000u) {
    // fp16 subnormal range [2^-24, 2^-14): m = RNE(|f| * 2^24); m == 1024
    // lands on the smallest normal, whose encoding is also 1024.
    const float scaled = bitcast::u32_to_f32(a) * 16777216.0f;
    return uint16_t(sign | uint16_t(std::nearbyint(scaled)));
  }
  // normal range: round the fp32 significand to 10 bits (RNE); a carry out of
  // the mantissa increments the exponent field, which is the right result.
  const uint32_t bias = 0xFFFu + ((a >> 13) & 1u);
  const uint32_t r = ((a + bias) >> 13) - (112u << 10);
  if (r >= 0x7C00u) return uint16_t(sign | 0x7C00u);
  return uint16_t(sign | r);
}

}  // namespace host_convert

}  // namespace inferop
