// Device introspection and the on-device self-test of the E4M3 conversions.
#include <stdio.h>
#include <string.h>

#include "device_common.h"
#include "hip_launch.h"

using namespace inferop_hip;

extern "C" int inferop_hip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n < 0) return 0;
  return n;
}

extern "C" int inferop_hip_current_device(int* ordinal) { return hipGetDevice(ordinal); }

extern "C" int inferop_hip_device_info(int ordinal, char* name, int name_len, int* arch,
                                       int* cu_count) {
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, ordinal);
  if (e != hipSuccess) return e;
  if (name && name_len > 0) snprintf(name, (size_t)name_len, "%s", p.name);
  if (arch) {
    // gcnArchName looks like "gfx950:sramecc+:xnack-"; its digits read as
    // hexadecimal (gfx950 -> 0x950, gfx90a -> 0x90a).
    int v = -1;
    if (strncmp(p.gcnArchName, "gfx", 3) == 0) {
      v = 0;
      for (const char* s = p.gcnArchName + 3; *s && *s != ':'; ++s) {
        if (*s >= '0' && *s <= '9') v = v * 16 + (*s - '0');
        else if (*s >= 'a' && *s <= 'f') v = v * 16 + (*s - 'a' + 10);
        else break;
      }
    }
    *arch = v;
  }
  if (cu_count) *cu_count = p.multiProcessorCount;
  return hipSuccess;
}

namespace {

// One fp32 bit pattern per thread.  Per-block partial results are combined
// with one 64-bit atomic per block and counter.
__global__ __launch_bounds__(256) void codec_selftest_kernel(uint64_t lo, uint64_t hi,
                                                             unsigned long long* counts) {
  __shared__ unsigned long long s_in, s_out, s_sum;
  if (threadIdx.x == 0) {
    s_in = 0;
    s_out = 0;
    s_sum = 0;
  }
  __syncthreads();
  unsigned long long in_dom = 0, out_dom = 0, sum = 0;
  const uint64_t stride = (uint64_t)gridDim.x * 256 * 4;
  for (uint64_t base = lo + ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4; base < hi; base += stride) {
    float v[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] = u2f((uint32_t)(base + t < hi ? base + t : base));
    const uint32_t hw = cvt_pk4_e4m3(v[0], v[1], v[2], v[3]);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint64_t i = base + t;
      if (i >= hi) break;
      const uint32_t sw = sw_e4m3(v[t]);
      const uint32_t hb = (hw >> (8 * t)) & 0xFFu;
      const uint32_t a = f2u(v[t]) & 0x7FFFFFFFu;
      const bool domain = a < 0x43E80000u;  // finite and |v| < 464
      if (hb != sw) {
        if (domain) ++in_dom;
        else ++out_dom;
      }
      sum += (unsigned long long)sw * (unsigned long long)(uint32_t)(i * 2654435761ull);
    }
  }
  atomicAdd(&s_in, in_dom);
  atomicAdd(&s_out, out_dom);
  atomicAdd(&s_sum, sum);
  __syncthreads();
  if (threadIdx.x == 0) {
    atomicAdd(counts + 0, s_in);
    atomicAdd(counts + 1, s_out);
    atomicAdd(counts + 2, s_sum);
  }
}

__global__ void decode_selftest_kernel(unsigned long long* counts) {
  const uint32_t b = threadIdx.x;  // 256 threads: one byte each
  const f32x2 hw = cvt_pk2_e4m3_f32<false>(b);
  const float sw = inferop::fp8::e4m3_to_float((uint8_t)b);
  const bool same = (hw.x != hw.x) ? (sw != sw) : (f2u(hw.x) == f2u(sw));
  if (!same) atomicAdd(counts + 3, 1ull);
}

}  // namespace

extern "C" int inferop_hip_selftest_fp8_codec(uint64_t lo, uint64_t hi, uint64_t* counts,
                                              void* stream) {
  if (hi > (1ull << 32) || lo > hi || !counts) return hipErrorInvalidValue;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint64_t n = hi - lo;
  uint64_t blocks = (n + 1023) / 1024;
  if (blocks > 65536) blocks = 65536;
  if (blocks == 0) blocks = 1;
  hipLaunchKernelGGL(codec_selftest_kernel, dim3((unsigned)blocks), dim3(256), 0, st, lo, hi,
                     (unsigned long long*)counts);
  hipLaunchKernelGGL(decode_selftest_kernel, dim3(1), dim3(256), 0, st,
                     (unsigned long long*)counts);
  return hipGetLastError();
}

// ---- measurement kernels (bench ceilings; no counterpart in the reference) ----

namespace {

// A plain read of n16 16-byte words: 256 lanes per workgroup, four
// non-temporal 16-byte loads in flight per lane (a wave reads 1 KB contiguous
// per load instruction), grid-striding over 16 KB chunks.  The loaded words
// feed a XOR that is stored only when it equals `magic`, so the loads cannot
// be dropped; the store is harmless either way (sink is scratch).
__global__ __launch_bounds__(256) void read_stream_kernel(const u32x4* __restrict__ p, int64_t n16,
                                                          uint32_t magic, uint32_t* sink) {
  uint32_t x = 0;
  const int64_t stride = (int64_t)gridDim.x * 1024;
  for (int64_t base = (int64_t)blockIdx.x * 1024; base < n16; base += stride) {
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = base + j * 256 + threadIdx.x;
      v[j] = i < n16 ? __builtin_nontemporal_load(p + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) x ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  if (x == magic) sink[0] = x;
}

typedef int i32x8_t __attribute__((ext_vector_type(8)));

// The prefill GEMM's inner loop without memory, shaped as one wave's share of
// a 256x256 tile per scale group: 8 weight slices x 4 activation slices, 32
// v_mfma_scale_f32_16x16x128_f8f6f4 (E4M3 x E4M3, 65536 flops each) per
// iteration; with PROMOTE each MFMA starts from zero and its four results are
// added to fp32 accumulators with the block scale (acc = fma(partial, s, acc),
// the GEMM's promotion), otherwise the MFMA accumulates in place.  Operands
// live in registers and are opaque to the compiler in every iteration (the
// asm statements emit no instruction), so nothing is hoisted out of the loop.
template <bool PROMOTE>
__global__ __launch_bounds__(256) void mfma_loop_kernel(int iters, uint32_t magic, uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  i32x8_t w[8], x[4];
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) w[t][e] = 0x38383838 ^ ((lane + t + e) & 0x03030303);
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) x[t][e] = 0x30303030 + t + e;
  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float sc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sc[j] = 1.0f + (lane + j) * 1e-7f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int t = 0; t < 8; ++t) asm volatile("" : "+v"(w[t]));
#pragma unroll
    for (int t = 0; t < 4; ++t) asm volatile("" : "+v"(x[t]));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (PROMOTE) {
          const f32x4 pv = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              w[i], x[j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(pv[r], sc[j], acc[i][j][r]);
        } else {
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w[i], x[j], acc[i][j], 0, 0,
                                                                       0, 127, 0, 127);
        }
      }
    }
  }
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) t += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
  if (__builtin_bit_cast(uint32_t, t) == magic) sink[0] = magic;
}

// One read of a [n, k] byte matrix by one workgroup of 8 waves per 16-row
// stripe, every load of the workgroup in flight at once (wave w takes scale
// groups [w*G, w*G + G) of the stripe's 16 rows, G = k / 1024), in one of the
// access patterns the decode GEMM kernels could use:
//   0: register loads, each instruction 8 rows x 128 B (the decode kernels'
//      row pattern: 8 lanes per 128-byte row segment)
//   1: register loads, each instruction 1 KB contiguous
//   2: register loads in the MFMA operand layout (lane l: row l % 16, 16 bytes
//      at chunk l / 16 of the group, then chunk l / 16 + 4): 16 rows x 64 B
//      per instruction
//   3: direct global->LDS loads, 8 rows x 128 B per instruction (the decode
//      kernels' loads), read back from LDS after one wait
//   4: pattern 0's register loads written to LDS (ds_write_b128, the layout
//      pattern 3 leaves) and read back, i.e. the register path into LDS
// With `stripes` > 0 workgroup b reads stripe b % stripes, so the data stays
// in L2 after the first touch and the launch measures a CU's load throughput
// rather than HBM.  The loaded words feed a XOR stored only when it equals
// `magic` (never, in practice), so no load can be dropped.
template <int P, int G>
__global__ __launch_bounds__(512) void stripe_read_kernel(const uint8_t* __restrict__ b, int k,
                                                          int stripes, uint32_t magic,
                                                          uint32_t* sink) {
  constexpr int L = 2 * G;  // 1 KB loads per wave
  __shared__ __attribute__((aligned(1024))) uint8_t lds[P >= 3 ? 8 * L * 1024 : 16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int sidx = stripes > 0 ? (int)(blockIdx.x % (unsigned)stripes) : (int)blockIdx.x;
  const uint8_t* s = b + (int64_t)sidx * 16 * k;
  u32x4 v[L];
  if constexpr (P == 0 || P == 3 || P == 4) {
    const int lrow = lane >> 3, ch = lane & 7;
    if constexpr (P == 4) {
#pragma unroll
      for (int i = 0; i < G; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          v[2 * i + h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
              s + (8 * h + lrow) * k + (w * G + i) * 128 + (ch ^ lrow) * 16));
#pragma unroll
      for (int i = 0; i < L; ++i)
        *reinterpret_cast<u32x4*>(lds + (w * L + i) * 1024 + lane * 16) = v[i];
      __syncthreads();
#pragma unroll
      for (int i = 0; i < L; ++i)
        v[i] = *reinterpret_cast<const u32x4*>(lds + (w * L + (i + 1) % L) * 1024 + lane * 16);
    } else if constexpr (P == 0) {
#pragma unroll
      for (int i = 0; i < G; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          v[2 * i + h] = __builtin_nontemporal_load(
              reinterpret_cast<const u32x4*>(s + (8 * h + lrow) * k + (w * G + i) * 128 + ch * 16));
    } else {
      const __amdgpu_buffer_rsrc_t r =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(s), (short)0, 16 * k, 0x00020000);
#pragma unroll
      for (int i = 0; i < G; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              r, (__attribute__((address_space(3))) void*)(lds + (w * L + 2 * i + h) * 1024), 16,
              (8 * h + lrow) * k + (w * G + i) * 128 + (ch ^ lrow) * 16, 0, 0, 2);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < L; ++i)
        v[i] = *reinterpret_cast<const u32x4*>(lds + (w * L + i) * 1024 + lane * 16);
    }
  } else if constexpr (P == 1) {
#pragma unroll
    for (int i = 0; i < L; ++i)
      v[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(s + (int64_t)(i * 8 + w) * 1024 + lane * 16));
  } else {
    const int r = lane & 15, c0 = lane >> 4;
#pragma unroll
    for (int i = 0; i < G; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        v[2 * i + h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            s + r * k + (w * G + i) * 128 + (c0 + 4 * h) * 16));
  }
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < L; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  if (x == magic) sink[0] = x;
}

template <int G>
hipError_t launch_stripe_read(int pattern, const uint8_t* b, int64_t n, int64_t k, int stripes,
                              uint32_t* sink, hipStream_t st) {
  const dim3 grid((unsigned)(n / 16)), block(512);
  const uint32_t magic = 0x9E3779B9u;
  switch (pattern) {
    case 0: hipLaunchKernelGGL((stripe_read_kernel<0, G>), grid, block, 0, st, b, (int)k, stripes, magic, sink); break;
    case 1: hipLaunchKernelGGL((stripe_read_kernel<1, G>), grid, block, 0, st, b, (int)k, stripes, magic, sink); break;
    case 2: hipLaunchKernelGGL((stripe_read_kernel<2, G>), grid, block, 0, st, b, (int)k, stripes, magic, sink); break;
    case 3: hipLaunchKernelGGL((stripe_read_kernel<3, G>), grid, block, 0, st, b, (int)k, stripes, magic, sink); break;
    default: hipLaunchKernelGGL((stripe_read_kernel<4, G>), grid, block, 0, st, b, (int)k, stripes, magic, sink); break;
  }
  return hipGetLastError();
}

}  // namespace

extern "C" int inferop_hip_diag_stripe_read(const void* b, int64_t n, int64_t k, int32_t pattern,
                                            int32_t stripes, uint32_t* sink, void* stream) {
  // one workgroup per 16 rows, G = k / 1024 groups of 128 bytes per wave
  if (!b || !sink || n < 16 || n % 16 != 0 || n / 16 > 65535 || k % 1024 != 0 || pattern < 0 ||
      pattern > 4 || stripes < 0 || (stripes > 0 && stripes > n / 16) || 16 * k > 0x7FFFFFFF)
    return hipErrorInvalidValue;
  const auto u8 = static_cast<const uint8_t*>(b);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (k / 1024) {
    case 2: return launch_stripe_read<2>(pattern, u8, n, k, stripes, sink, st);
    case 7: return launch_stripe_read<7>(pattern, u8, n, k, stripes, sink, st);
    case 8: return launch_stripe_read<8>(pattern, u8, n, k, stripes, sink, st);
    default: return hipErrorInvalidValue;
  }
}

extern "C" int inferop_hip_diag_read_stream(const void* src, int64_t bytes, int32_t blocks,
                                            uint32_t* sink, void* stream) {
  if (!src || !sink || bytes < 16 || bytes % 16 != 0 || blocks < 1 || blocks > (1 << 20))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(read_stream_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(src), bytes / 16,
                     0x9E3779B9u, sink);
  return hipGetLastError();
}

extern "C" int inferop_hip_diag_mfma_loop(int32_t iters, int32_t blocks, int32_t promote,
                                          uint32_t* sink, void* stream) {
  if (!sink || iters < 1 || blocks < 1 || blocks > (1 << 20)) return hipErrorInvalidValue;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (promote) {
    hipLaunchKernelGGL(mfma_loop_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, st, iters,
                       0x7F7FFFFFu, sink);
  } else {
    hipLaunchKernelGGL(mfma_loop_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, st, iters,
                       0x7F7FFFFFu, sink);
  }
  return hipGetLastError();
}
