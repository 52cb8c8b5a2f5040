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
// order, DPP within rows); the probabilities go through LDS so that every
// lane adds them in index order, which is what makes l -- and so every weight --
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
__global__ __launch_bounds__(64) void topk_softmax_kernel(int32_t* __restrict__ ids,
                                                           float* __restrict__ weights,
                                                           const float* __restrict__ logits,
                                                           int tokens, int num_experts, int topk,
                                                           int renormalize) {
  // one wave (one token) per workgroup: at 64 tokens four tokens per
  // workgroup took 6.1 us against 5.5 us, at 4096 tokens the two are level
  __shared__ __attribute__((aligned(16))) float sp[kMaxExperts];
  const int lane = threadIdx.x;
  const int t = blockIdx.x;
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
    sp[e] = e < num_experts ? p[j] : 0.0f;  // slots past the last expert add +0
  }
  // l = p[0] + p[1] + ... in index order (the reference's left-to-right sum),
  // the same chain in every lane from broadcast LDS reads: the slots past the
  // last expert hold +0 (l >= +0, so adding them changes nothing), and the
  // reads of the next 8 slots are issued before the adds of the current 8, so
  // the LDS latency is not waited out per batch
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float l = 0.0f;
  {
    constexpr int kB = 8;                // f32x4 reads per batch
    constexpr int kN = EPL * 64 / 4;     // f32x4 slots covering EPL * 64 experts
    constexpr int kBatches = (kN + kB - 1) / kB;
    const f32x4* q4 = reinterpret_cast<const f32x4*>(&sp[0]);
    f32x4 cur[kB], nxt[kB];
#pragma unroll
    for (int i = 0; i < kB; ++i) cur[i] = i < kN ? q4[i] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < kBatches; ++b) {
      if (b + 1 < kBatches) {
#pragma unroll
        for (int i = 0; i < kB; ++i) {
          const int q = (b + 1) * kB + i;
          nxt[i] = q < kN ? q4[q] : f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
      for (int i = 0; i < kB; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) l += cur[i][r];
      }
#pragma unroll
      for (int i = 0; i < kB; ++i) cur[i] = nxt[i];
    }
  }

  // top-k in the reference's order (probability descending, lower index
  // first).  p >= 0, so its bits order like its value; a lane keeps each of
  // its experts as key bits + 1 (0 = taken or past the last expert).  A round
  // takes the largest key in the wave; among lanes holding it the lowest
  // expert is the lowest lane at the lowest slot j (expert = lane + 64 j),
  // found with one ballot per slot (or a single ballot when one lane holds
  // it), and that lane clears the slot.
  uint32_t key[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) key[j] = (lane + 64 * j < num_experts) ? f2u(p[j]) + 1u : 0u;
  int32_t* tid = ids + (int64_t)t * topk;
  float* tw = weights + (int64_t)t * topk;
  uint32_t my_b = 0;  // lane k < 64: bits of choice k's probability
  int32_t my_id = 0;
  float wsum_big = 0.0f;  // topk > 64: the weights' left-to-right sum
  for (int k = 0; k < topk; ++k) {
    uint32_t best = key[0];
    int jb = 0;
#pragma unroll
    for (int j = 1; j < EPL; ++j)
      if (key[j] > best) best = key[j], jb = j;  // first slot on ties
    const uint32_t bb = wave_max_u32(best);
    // with four or more slots per lane, one ballot first: one lane holds the
    // maximum in the usual case (256 experts, 64 tokens: 5.5 -> 5.1 us; 1024
    // experts 19.1 -> 12.7 us); with one or two slots the per-slot ballots
    // cost less than the test
    const uint64_t held = EPL >= 4 ? __builtin_amdgcn_ballot_w64(best == bb) : 0;
    int be;
    if (EPL >= 4 && __builtin_popcountll(held) == 1) {
      be = __builtin_amdgcn_readlane(lane + 64 * jb, (int)__builtin_ctzll(held));
    } else {
      be = 0x7FFFFFFF;
#pragma unroll
      for (int j = EPL - 1; j >= 0; --j) {
        const uint64_t m = __builtin_amdgcn_ballot_w64(best == bb && jb == j);
        if (m) be = (int)__builtin_ctzll(m) + 64 * j;  // lowest slot wins: taken last
      }
    }
    if (lane == (be & 63)) {
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        if (j == (be >> 6)) key[j] = 0u;
    }
    if (topk <= 64) {
      if (lane == k) my_b = bb - 1u, my_id = be;
    } else {
      const float wk = u2f(bb - 1u) / l;
      if (lane == 0) tid[k] = be, tw[k] = wk;
      wsum_big += wk;
    }
  }
  if (topk <= 64) {
    // weights p / l, then their left-to-right sum for renormalize
    const float my_w = u2f(my_b) / l;
    float wsum = 0.0f;
    for (int k = 0; k < topk; ++k)
      wsum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_w), k));
    const bool renorm = renormalize && wsum > 0.0f;
    if (lane < topk) {
      tid[lane] = my_id;
      tw[lane] = renorm ? my_w / wsum : my_w;
    }
  } else if (renormalize && wsum_big > 0.0f && lane == 0) {
    for (int k = 0; k < topk; ++k) tw[k] = tw[k] / wsum_big;
  }
}

template <int EPL>
hipError_t launch_topk(int32_t* ids, float* weights, const float* logits, int tokens, int e, int k,
                       int renorm, hipStream_t st) {
  hipLaunchKernelGGL((topk_softmax_kernel<EPL>), dim3((unsigned)tokens), dim3(64), 0,
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
