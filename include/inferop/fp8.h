// inferop (MI355X build) : OCP E4M3FN codec, host and device.
//
// Drop-in for the reference header include/inferop/fp8.h (fp8.h:24,40-96):
// same names, same results for every input.  The format is OCP FP8 E4M3FN:
// bias 7, no infinities, S.1111.111 is NaN, largest finite value 448,
// subnormals m * 2^-9.  Encoding rounds to nearest-even and saturates
// (SATFINITE): NaN -> S|0x7F, +-Inf and |f| >= 464 -> S|0x7E (+-448),
// |f| <= 2^-10 -> signed zero.
//
// The encoder below works on the fp32 bit pattern: a rounding bias added to
// the magnitude bits rounds the 23-bit fraction to 3 bits (a carry into the
// exponent field is the correct result), and the E4M3 subnormal band is
// rounded with rint() on |f| * 2^9.  It is checked against an independent
// nearest-grid-point encoder over all 2^32 inputs by the test-suite.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

#if defined(__HIPCC__)
#define INFEROP_HD __host__ __device__
#else
#define INFEROP_HD
#endif

namespace inferop {
namespace fp8 {

constexpr float kE4M3Max = 448.0f;

namespace detail {
INFEROP_HD inline uint32_t bits_of(float f) {
  uint32_t w;
  memcpy(&w, &f, 4);
  return w;
}
INFEROP_HD inline float float_of(uint32_t w) {
  float f;
  memcpy(&f, &w, 4);
  return f;
}
}  // namespace detail

// Exact decode of any byte; 0x7F / 0xFF decode to a quiet NaN carrying the sign.
INFEROP_HD inline float e4m3_to_float(uint8_t b) {
  const uint32_t sign = uint32_t(b & 0x80u) << 24;
  const uint32_t em = b & 0x7Fu;
  if (em == 0x7Fu) return detail::float_of(sign | 0x7FC00000u);
  if (em < 0x08u) {
    // subnormal or zero: m * 2^-9 is exact in fp32.
    return detail::float_of(sign | detail::bits_of(float(em) * 0.001953125f));
  }
  // normal: exponent field E in [1, 15] re-biased by 127 - 7 = 120; the
  // three mantissa bits move to the top of the fp32 fraction.
  return detail::float_of(sign | ((em + (120u << 3)) << 20));
}

// Round-to-nearest-even, saturating encode (OCP SATFINITE).
INFEROP_HD inline uint8_t float_to_e4m3_rn_sat(float f) {
  const uint32_t w = detail::bits_of(f);
  const uint32_t sign = (w >> 24) & 0x80u;
  const uint32_t a = w & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return uint8_t(sign | 0x7Fu);   // NaN
  if (a >= 0x43E80000u) return uint8_t(sign | 0x7Eu);  // |f| >= 464 (RNE tie goes to 448), Inf
  if (a < 0x3C800000u) {
    // below the smallest normal 2^-6: the E4M3 subnormal grid is k * 2^-9,
    // k = rint(|f| * 512) in [0, 8]; k == 8 is the encoding of 2^-6 itself.
    const float k = rintf(detail::float_of(a) * 512.0f);
    return uint8_t(sign | uint32_t(k));
  }
  // normal: keep 3 fraction bits with round-to-nearest-even.
  const uint32_t bias = 0x7FFFFu + ((a >> 20) & 1u);
  const uint32_t code = ((a + bias) >> 20) - (120u << 3);
  return uint8_t(sign | code);
}

}  // namespace fp8
}  // namespace inferop
