// TEST INFRASTRUCTURE ONLY: extern "C" bindings over the reference's own CPU
// golden code (reference/reference.cpp and include/inferop/{fp8,common}.h of
// TheonHuang/Inference), compiled from the reference sources where they lie by
// oracle/Makefile into oracle/_ref/libinferop_ref.so.  Used to check the
// oracle restatement and to write the golden fixtures; never shipped.
#include <cstdint>
#include <cstring>

#include "inferop/common.h"
#include "inferop/fp8.h"
#include "reference.h"

extern "C" {

uint8_t ref_float_to_e4m3(float f) { return inferop::fp8::float_to_e4m3_rn_sat(f); }
float ref_e4m3_to_float(uint8_t b) { return inferop::fp8::e4m3_to_float(b); }
uint16_t ref_float_to_bf16(float f) { return inferop::host_convert::float_to_bf16_rn(f); }
float ref_bf16_to_float(uint16_t v) { return inferop::host_convert::bf16_to_float(v); }
uint16_t ref_float_to_half(float f) { return inferop::host_convert::float_to_half_rn(f); }
float ref_half_to_float(uint16_t h) { return inferop::host_convert::half_to_float(h); }

// Exhaustive helpers: write the reference's encode of every fp32 bit pattern
// in [lo, hi) into out[0 .. hi-lo).
void ref_encode_range(uint64_t lo, uint64_t hi, uint8_t* out) {
  for (uint64_t i = lo; i < hi; ++i) {
    uint32_t w = uint32_t(i);
    float f;
    std::memcpy(&f, &w, 4);
    out[i - lo] = inferop::fp8::float_to_e4m3_rn_sat(f);
  }
}
void ref_bf16_range(uint64_t lo, uint64_t hi, uint16_t* out) {
  for (uint64_t i = lo; i < hi; ++i) {
    uint32_t w = uint32_t(i);
    float f;
    std::memcpy(&f, &w, 4);
    out[i - lo] = inferop::host_convert::float_to_bf16_rn(f);
  }
}
void ref_half_range(uint64_t lo, uint64_t hi, uint16_t* out) {
  for (uint64_t i = lo; i < hi; ++i) {
    uint32_t w = uint32_t(i);
    float f;
    std::memcpy(&f, &w, 4);
    out[i - lo] = inferop::host_convert::float_to_half_rn(f);
  }
}

void ref_quant(uint8_t* q, float* scales, const float* x, int64_t rows, int64_t cols, int gs) {
  inferop::ref::quant_fp8_per_token_group(q, scales, x, rows, cols, gs);
}
void ref_dequant(float* x, const uint8_t* q, const float* scales, int64_t rows, int64_t cols,
                 int gs) {
  inferop::ref::dequant_fp8_per_token_group(x, q, scales, rows, cols, gs);
}
void ref_gemm(float* c, const uint8_t* a_q, const float* a_scales, const uint8_t* b_q,
              const float* b_scales, int64_t m, int64_t n, int64_t k, int gs, int bn) {
  inferop::ref::w8a8_block_fp8_gemm(c, a_q, a_scales, b_q, b_scales, m, n, k, gs, bn);
}

void ref_rmsnorm(float* out, const float* in, const float* w, int64_t rows, int64_t cols,
                 float eps) {
  inferop::ref::rmsnorm(out, in, w, rows, cols, eps);
}
void ref_fused_add_rmsnorm(float* residual, float* out, const float* x, const float* w,
                           int64_t rows, int64_t cols, float eps) {
  inferop::ref::fused_add_rmsnorm(residual, out, x, w, rows, cols, eps);
}
void ref_silu_and_mul(float* out, const float* gate_up, int64_t tokens, int64_t d) {
  inferop::ref::silu_and_mul(out, gate_up, tokens, d);
}

void ref_topk_softmax(int32_t* ids, float* w, const float* logits, int64_t tokens, int experts,
                      int topk, int renormalize) {
  inferop::ref::topk_softmax(ids, w, logits, tokens, experts, topk, renormalize != 0);
}

}  // extern "C"
