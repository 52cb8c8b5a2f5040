// Device helpers shared by the gfx950 kernels: E4M3 conversions, 16-lane
// DPP-row reductions, output-dtype stores.  Compiled by hipcc only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "inferop/fp8.h"

namespace inferop_hip {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// dtype tags of the public ABI (inferop::dtype values).
enum : int32_t { kFp32 = 0, kFp16 = 1, kBf16 = 2, kFp8 = 3 };

__device__ __forceinline__ uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// ---- 16-lane row reduction (one DPP row == one 128-element group) ----------
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror: after
// the four steps every lane of the row holds the row maximum.
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  return v;
}

// ---- E4M3 encode ------------------------------------------------------------
// Hardware path: v_cvt_pk_fp8_f32 (OCP E4M3 on gfx950, round-to-nearest-even).
// Used only on values the quantizer's fast path can produce (finite,
// |v| < 464); its agreement with the software encoder on that whole domain is
// checked exhaustively on the device by inferop_selftest_fp8_codec.
__device__ __forceinline__ uint32_t cvt_pk4_e4m3(float a, float b, float c, float d) {
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
}

// Software path: the exact reference semantics (include/inferop/fp8.h).
__device__ __forceinline__ uint32_t sw_e4m3(float v) {
  return inferop::fp8::float_to_e4m3_rn_sat(v);
}

// ---- E4M3 decode --------------------------------------------------------------
// v_cvt_pk_f32_fp8: exact for every finite byte; checked on all 256 bytes.
template <bool HI>
__device__ __forceinline__ f32x2 cvt_pk2_e4m3_f32(uint32_t w) {
  return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, HI);
}

// ---- output conversions ---------------------------------------------------------
// bf16 / fp16 stores round to nearest-even (v_cvt_pk_bf16_f32, v_cvt_f16_f32),
// the conversions the reference's kernels use (__float2bfloat16, __float2half).

// x as an fp32 register the optimiser cannot see through.  Narrowing an fp32
// product to fp16 is otherwise folded into one mixed-precision FMA
// (v_fma_mixlo_f16 a, b, 0), which rounds the exact product to fp16 once;
// the C semantics, and the reference, round it to fp32 first, and the two
// differ where the fp32 rounding lands on an fp16 tie.  Every fp32 -> fp16
// conversion of a computed value goes through this.
__device__ __forceinline__ float fp32_value(float x) {
  asm("" : "+v"(x));
  return x;
}
__device__ __forceinline__ _Float16 to_fp16(float x) { return (_Float16)fp32_value(x); }
template <int OUT_DT>
struct OutT;
template <>
struct OutT<kFp32> {
  using T = float;
};
template <>
struct OutT<kFp16> {
  using T = _Float16;
};
template <>
struct OutT<kBf16> {
  using T = __bf16;
};

// An fp32 result as the output type (fp16 through to_fp16).
template <int OUT_DT>
__device__ __forceinline__ typename OutT<OUT_DT>::T to_out(float x) {
  if constexpr (OUT_DT == kFp16)
    return to_fp16(x);
  else
    return (typename OutT<OUT_DT>::T)x;
}

// Store 4 consecutive outputs (row-major, 4-element aligned) as one vector.
template <int OUT_DT>
__device__ __forceinline__ void store4(void* dst, float a, float b, float c, float d) {
  if constexpr (OUT_DT == kFp32) {
    *reinterpret_cast<f32x4*>(dst) = f32x4{a, b, c, d};
  } else if constexpr (OUT_DT == kBf16) {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<bf16x4*>(dst) = bf16x4{(__bf16)a, (__bf16)b, (__bf16)c, (__bf16)d};
  } else {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<f16x4*>(dst) = f16x4{to_fp16(a), to_fp16(b), to_fp16(c), to_fp16(d)};
  }
}

template <int OUT_DT>
__device__ __forceinline__ void store1(void* dst, float a) {
  if constexpr (OUT_DT == kFp16)
    *reinterpret_cast<_Float16*>(dst) = to_fp16(a);
  else
    *reinterpret_cast<typename OutT<OUT_DT>::T*>(dst) = (typename OutT<OUT_DT>::T)a;
}

}  // namespace inferop_hip
