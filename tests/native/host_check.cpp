// TEST HELPER: exposes the product's host-side headers (include/inferop/fp8.h,
// include/inferop/common.h) and the quantizer's quotient arithmetic
// (inferop_amd/csrc/quant_math.h) to the Python tests, for exhaustive
// comparison with the oracle and the compiled reference.
#include <cstdint>
#include <cstring>

#include "inferop/common.h"
#include "inferop/fp8.h"
#include "quant_math.h"

namespace {
inline float f_of(uint32_t w) {
  float f;
  std::memcpy(&f, &w, 4);
  return f;
}
inline uint32_t b_of(float f) {
  uint32_t w;
  std::memcpy(&w, &f, 4);
  return w;
}
}  // namespace

extern "C" {

void hc_encode_range(uint64_t lo, uint64_t hi, uint8_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = int64_t(lo); i < int64_t(hi); ++i)
    out[i - int64_t(lo)] = inferop::fp8::float_to_e4m3_rn_sat(f_of(uint32_t(i)));
}

float hc_decode(uint8_t b) { return inferop::fp8::e4m3_to_float(b); }

void hc_bf16_range(uint64_t lo, uint64_t hi, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = int64_t(lo); i < int64_t(hi); ++i)
    out[i - int64_t(lo)] = inferop::host_convert::float_to_bf16_rn(f_of(uint32_t(i)));
}

void hc_half_range(uint64_t lo, uint64_t hi, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = int64_t(lo); i < int64_t(hi); ++i)
    out[i - int64_t(lo)] = inferop::host_convert::float_to_half_rn(f_of(uint32_t(i)));
}

float hc_half_to_float(uint16_t h) { return inferop::host_convert::half_to_float(h); }
float hc_bf16_to_float(uint16_t h) { return inferop::host_convert::bf16_to_float(h); }

// Exhaustive proof of the quantizer fast-path quotient for 16-bit inputs.
// kind 0: bf16, kind 1: fp16.  For every finite positive absmax the fast path
// admits (bf16: absmax >= 2^-80; fp16: all) and every finite x of the same
// type with |x| <= absmax, compare div_by_recip(x, s, RN(1/s)) with the IEEE
// quotient x / s bitwise, s = absmax * fl32(1/448).  The all-zero group
// (s = 1, x = +-0) is included.  out[0] = pairs checked, out[1] = quotient
// mismatches, out[2] = E4M3 byte mismatches, out[3] = quotient mismatches
// with |x/s| >= 2^-11.  (Quotient mismatches occur only where x or x/s is in
// the fp32 subnormal range, where the residual x - q0*s or the quotient is
// rounded to the subnormal grid; those quotients are far below 2^-10 and
// encode to a signed zero either way.)
void hc_markstein_sweep(int kind, uint64_t* out) {
  const float inv448 = inferop_qmath::kInv448;
  uint64_t pairs = 0, bad = 0, bad_bytes = 0, bad_normal = 0;
  const uint32_t top = kind == 0 ? 0x7F80u : 0x7C00u;  // first non-finite magnitude
  auto to_f = [kind](uint32_t h) -> float {
    if (kind == 0) return inferop::host_convert::bf16_to_float(uint16_t(h));
    return inferop::host_convert::half_to_float(uint16_t(h));
  };
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, bad, bad_bytes, bad_normal)
  for (int64_t am = 0; am < int64_t(top); ++am) {
    const float amax = to_f(uint32_t(am));
    if (am != 0 && kind == 0 && b_of(amax) < inferop_qmath::kFastMinAbsmaxBits) continue;  // slow path
    const float s = am == 0 ? 1.0f : amax * inv448;
    const float r = 1.0f / s;
    for (uint32_t xm = 0; xm <= uint32_t(am); ++xm) {
      for (uint32_t sg = 0; sg < 2; ++sg) {
        const float x = to_f(xm | (sg << 15));
        volatile float ieee = x / s;
        const float fast = inferop_qmath::div_by_recip(x, s, r);
        ++pairs;
        if (b_of(fast) != b_of(ieee)) {
          ++bad;
          if ((b_of(ieee) & 0x7FFFFFFFu) >= 0x3A000000u) ++bad_normal;
          if (inferop::fp8::float_to_e4m3_rn_sat(fast) != inferop::fp8::float_to_e4m3_rn_sat(ieee))
            ++bad_bytes;
        }
      }
    }
  }
  out[0] = pairs;
  out[1] = bad;
  out[2] = bad_bytes;
  out[3] = bad_normal;
}

}  // extern "C"
