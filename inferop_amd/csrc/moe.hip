// MoE routing for gfx950: softmax over expert logits and top-k selection.
//
// Semantics (reference/reference.cpp:152-181): per token, mx = max logit,
// p[e] = exp(logit[e] - mx), l = p[0] + p[1] + ... left to right, experts
// ordered by p descending with the lower index first on ties, and the first
// topk of that order returned with weight p / l; with renormalize the weights
// are divided by their left-to-right sum (when it is positive).
//
// One wave per token.  The logits are read coalesced, each lane holding EPL
// experts; the max and every top-k argmax are wave reductions (exact in any
// order, DPP within rows); the probabilities go through LDS so that one lane
// adds them in index order, which is what makes l -- and so every weight --
// the reference's value.  exp is evaluated in double precision and
// rounded once to fp32 (the correctly rounded exponential except in rare
// last-bit cases, like the host's expf).
#include "device_common.h"
#include "hip_launch.h"

namespace inferop_hip {
namespace {

constexpr int kMaxExperts = 1024;

__device__ __forceinline__ uint32_t row16_min_u32(uint32_t v) {
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  return v;
}

// Wave-wide max / min: DPP within each 16-lane row, then the four rows.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = row16_max_u32(v);
  return max(max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
             max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = row16_min_u32(v);
  return min(min((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
             min((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
}

// Order-preserving map of a float to uint32 (NaN to 0: a NaN logit never
// becomes the maximum, as with std::max in the reference).
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t b = f2u(f);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float funkey(uint32_t k) {
  return u2f((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

template <int EPL>
__global__ __launch_bounds__(256) void topk_softmax_kernel(int32_t* __restrict__ ids,
                                                           float* __restrict__ weights,
                                                           const float* __restrict__ logits,
                                                           int tokens, int num_experts, int topk,
                                                           int renormalize) {
  __shared__ __attribute__((aligned(16))) float sp[4][kMaxExperts];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + w;
  if (t >= tokens) return;  // whole wave; no workgroup barrier follows
  const float* row = logits + (int64_t)t * num_experts;
  float x[EPL];
  uint32_t mk = 0;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    x[j] = e < num_experts ? row[e] : -__builtin_inff();
    mk = max(mk, fkey(x[j]));
  }
  const float mx = funkey(wave_max_u32(mk));
  float p[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    p[j] = (float)::exp((double)(x[j] - mx));
    if (e < num_experts) sp[w][e] = p[j];
  }
  // l = p[0] + p[1] + ... in index order (the reference's left-to-right sum):
  // one lane adds them from LDS, four at a time
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float l = 0.0f;
  if (lane == 0) {
    const f32x4* q4 = reinterpret_cast<const f32x4*>(&sp[w][0]);
    const int n4 = num_experts >> 2;
#pragma unroll 8
    for (int i = 0; i < n4; ++i) {
      const f32x4 v = q4[i];
      l += v[0];
      l += v[1];
      l += v[2];
      l += v[3];
    }
    for (int e = n4 << 2; e < num_experts; ++e) l += sp[w][e];
  }
  l = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, l)));

  // top-k in the reference's order (probability descending, lower index
  // first): p >= 0, so its bits order like its value; each pass takes the
  // largest probability among the experts after the last one chosen, then
  // the lowest index holding it
  int32_t* tid = ids + (int64_t)t * topk;
  float* tw = weights + (int64_t)t * topk;
  uint32_t prev_b = 0xFFFFFFFFu;  // above every probability
  int prev_e = -1;
  float wsum = 0.0f;
  int32_t my_id = 0;
  float my_w = 0.0f;
  for (int k = 0; k < topk; ++k) {
    uint32_t key = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = lane + 64 * j;
      const uint32_t b = f2u(p[j]);
      const bool after = b < prev_b || (b == prev_b && e > prev_e);
      if (e < num_experts && after) key = max(key, b + 1u);
    }
    const uint32_t bb = wave_max_u32(key) - 1u;  // the chosen probability's bits
    uint32_t ei = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = lane + 64 * j;
      const uint32_t b = f2u(p[j]);
      const bool after = b < prev_b || (b == prev_b && e > prev_e);
      if (e < num_experts && after && b == bb) ei = min(ei, (uint32_t)e);
    }
    const int be = (int)wave_min_u32(ei);
    prev_b = bb;
    prev_e = be;
    const float wk = u2f(bb) / l;
    if (topk <= 64) {
      // lane k keeps choice k; the row is stored once at the end
      if (lane == k) {
        my_id = be;
        my_w = wk;
      }
    } else if (lane == 0) {
      tid[k] = be;
      tw[k] = wk;
    }
    wsum += wk;  // every lane holds the same left-to-right sum
  }
  const bool renorm = renormalize && wsum > 0.0f;
  if (topk <= 64) {
    if (lane < topk) {
      tid[lane] = my_id;
      tw[lane] = renorm ? my_w / wsum : my_w;
    }
  } else if (renorm && lane == 0) {
    for (int k = 0; k < topk; ++k) tw[k] = tw[k] / wsum;
  }
}

template <int EPL>
hipError_t launch_topk(int32_t* ids, float* weights, const float* logits, int tokens, int e, int k,
                       int renorm, hipStream_t st) {
  hipLaunchKernelGGL((topk_softmax_kernel<EPL>), dim3((unsigned)((tokens + 3) / 4)), dim3(256), 0,
                     st, ids, weights, logits, tokens, e, k, renorm);
  return hipGetLastError();
}

}  // namespace
}  // namespace inferop_hip

using namespace inferop_hip;

extern "C" int inferop_hip_topk_softmax(int32_t* ids, float* weights, const float* logits,
                                        int tokens, int num_experts, int topk, int renormalize,
                                        void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (num_experts <= 64) return launch_topk<1>(ids, weights, logits, tokens, num_experts, topk, renormalize, st);
  if (num_experts <= 128) return launch_topk<2>(ids, weights, logits, tokens, num_experts, topk, renormalize, st);
  if (num_experts <= 256) return launch_topk<4>(ids, weights, logits, tokens, num_experts, topk, renormalize, st);
  if (num_experts <= 512) return launch_topk<8>(ids, weights, logits, tokens, num_experts, topk, renormalize, st);
  if (num_experts <= kMaxExperts)
    return launch_topk<16>(ids, weights, logits, tokens, num_experts, topk, renormalize, st);
  return hipErrorInvalidValue;
}
