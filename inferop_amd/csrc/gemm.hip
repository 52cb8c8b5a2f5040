// W8A8 blockwise-FP8 GEMM for gfx950 (CDNA4).
//
//   C[m,n] = sum_g sa[m,g] * sb[n/128,g] * sum_{k in group g} A[m,k] * B[n,k]
//   A: [M,K] E4M3, sa: [M,K/128] fp32, B: [N,K] E4M3, sb: [ceil(N/128),K/128] fp32
//
// Matrix cores: v_mfma_scale_f32_16x16x128_f8f6f4 with both formats E4M3 and
// unit E8M0 scales.  One instruction multiplies a 16x128 weight slice by a
// 16x128 activation slice, i.e. exactly one 128-wide scale group, so each
// MFMA yields the group's partial dot products exactly as the fp8 products
// sum in fp32; the fp32 block scales are then applied in VALU registers:
//   acc = fma(partial, sa[m,g] * sb[n/128,g], acc)
// The weight slice is the MFMA "A" operand and the activation slice the "B"
// operand, so a lane's four accumulator registers are four consecutive n of
// one output row m: one activation scale per lane per 16-row slice, and the
// weight scale is uniform across a wave (a wave never straddles a 128-row
// weight block) and lives in an SGPR.  The same four registers are four
// contiguous outputs in memory, stored as one vector.
//
// Data movement: a workgroup owns a BN x BM output tile (n x m).  Per scale
// group it stages B[BN,128] and A[BM,128] in LDS, double-buffered: the next
// group's global loads are in flight while the current group's MFMAs run.  An
// LDS row is 128 bytes = eight 16-byte chunks, stored at chunk ^ (row & 7) so
// the eight lanes of a ds_read_b128 phase hit eight different bank groups.
// Each lane feeds the MFMA with chunks (lane/16) and (lane/16 + 4) of its
// row; both operands use the same chunk order, so the K permutation cancels.
//
// Split-K (small M): blockIdx.z selects a range of scale groups.  Each split
// writes its fp32 partial tile to a library-owned workspace; the last split
// to arrive (device-scope atomic counter) adds the partials in split order,
// writes C and resets the counter, so results are deterministic and no block
// ever waits on another.
#include <mutex>
#include <unordered_map>

#include "device_common.h"
#include "hip_launch.h"

namespace inferop_hip {
namespace {

struct GemmArgs {
  void* c;
  const uint8_t* aq;
  const float* as;
  const uint8_t* bq;
  const float* bs;
  float* ws;      // split-K partials
  int* counters;  // split-K arrival counters, one per output tile
  int m, n, k;
  int split;
  int vec_ok;  // C rows can take 4-element vector stores (N % 4 == 0, C aligned)
};

__device__ __forceinline__ i32x8 lds_operand(const uint8_t* base, int row, int c0) {
  const uint8_t* r = base + row * 128;
  const int x = row & 7;
  const uint4 lo = *reinterpret_cast<const uint4*>(r + ((c0 ^ x) << 4));
  const uint4 hi = *reinterpret_cast<const uint4*>(r + ((c0 ^ x ^ 4) << 4));
  return i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
               (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

template <int BN, int BM, int WN, int WM, int OUT_DT, bool SPLIT>
__global__ __launch_bounds__(64 * WN * WM) void gemm_kernel(GemmArgs a) {
  constexpr int T = 64 * WN * WM;
  constexpr int TN = BN / WN, TM = BM / WM;
  constexpr int SN = TN / 16, SM = TM / 16;
  constexpr int CB = (BN * 8 + T - 1) / T;
  constexpr int CA = (BM * 8 + T - 1) / T;
  constexpr int kStage = (BN + BM) * 128;
  static_assert(TN % 16 == 0 && TM % 16 == 0, "wave tile must be a multiple of 16");
  static_assert(128 % TN == 0, "a wave must stay inside one 128-row weight block");

  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % WN, wm = wave / WN;
  const int M = a.m, N = a.n, K = a.k;
  const int KG = K >> 7;
  const int NB = (N + 127) >> 7;
  const int n0 = blockIdx.x * BN;
  const int m0 = blockIdx.y * BM;
  const int z = blockIdx.z;
  const int g_begin = (int)((int64_t)z * KG / a.split);
  const int g_end = (int)((int64_t)(z + 1) * KG / a.split);

  // global -> LDS staging slots (fixed per thread for the whole K loop)
  const uint8_t* srcB[CB];
  int ldsB[CB];
  const uint8_t* srcA[CA];
  int ldsA[CA];
#pragma unroll
  for (int s = 0; s < CB; ++s) {
    const int idx = tid + s * T;
    const int row = idx >> 3, c = idx & 7;
    const int grow = min(n0 + row, N - 1);
    srcB[s] = a.bq + (int64_t)grow * K + c * 16;
    ldsB[s] = (idx < BN * 8) ? row * 128 + ((c ^ (row & 7)) << 4) : -1;
  }
#pragma unroll
  for (int s = 0; s < CA; ++s) {
    const int idx = tid + s * T;
    const int row = idx >> 3, c = idx & 7;
    const int grow = min(m0 + row, M - 1);
    srcA[s] = a.aq + (int64_t)grow * K + c * 16;
    ldsA[s] = (idx < BM * 8) ? BN * 128 + row * 128 + ((c ^ (row & 7)) << 4) : -1;
  }

  // scale pointers: one activation row per lane per 16-row slice, one weight
  // block per wave.
  const float* saP[SM];
#pragma unroll
  for (int j = 0; j < SM; ++j) {
    const int mrow = min(m0 + wm * TM + 16 * j + (lane & 15), M - 1);
    saP[j] = a.as + (int64_t)mrow * KG;
  }
  const int nbw = min((n0 + wn * TN) >> 7, NB - 1);
  const float* sbP = a.bs + (int64_t)nbw * KG;

  f32x4 acc[SN][SM];
#pragma unroll
  for (int i = 0; i < SN; ++i)
#pragma unroll
    for (int j = 0; j < SM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint4 stB[CB], stA[CA];
  float saN[SM], sbN = 0.f;

  if (g_begin < g_end) {
#pragma unroll
    for (int s = 0; s < CB; ++s)
      if (ldsB[s] >= 0) stB[s] = *reinterpret_cast<const uint4*>(srcB[s] + g_begin * 128);
#pragma unroll
    for (int s = 0; s < CA; ++s)
      if (ldsA[s] >= 0) stA[s] = *reinterpret_cast<const uint4*>(srcA[s] + g_begin * 128);
#pragma unroll
    for (int j = 0; j < SM; ++j) saN[j] = saP[j][g_begin];
    sbN = sbP[g_begin];
#pragma unroll
    for (int s = 0; s < CB; ++s)
      if (ldsB[s] >= 0) *reinterpret_cast<uint4*>(smem + ldsB[s]) = stB[s];
#pragma unroll
    for (int s = 0; s < CA; ++s)
      if (ldsA[s] >= 0) *reinterpret_cast<uint4*>(smem + ldsA[s]) = stA[s];
  }
  __syncthreads();

  const int c0 = lane >> 4;
  const int rsub = lane & 15;
  int buf = 0;
  for (int g = g_begin; g < g_end; ++g) {
    float saC[SM];
#pragma unroll
    for (int j = 0; j < SM; ++j) saC[j] = saN[j];
    const float sbC = sbN;
    const bool more = g + 1 < g_end;
    if (more) {
#pragma unroll
      for (int s = 0; s < CB; ++s)
        if (ldsB[s] >= 0) stB[s] = *reinterpret_cast<const uint4*>(srcB[s] + (g + 1) * 128);
#pragma unroll
      for (int s = 0; s < CA; ++s)
        if (ldsA[s] >= 0) stA[s] = *reinterpret_cast<const uint4*>(srcA[s] + (g + 1) * 128);
#pragma unroll
      for (int j = 0; j < SM; ++j) saN[j] = saP[j][g + 1];
      sbN = sbP[g + 1];
    }

    const uint8_t* bB = smem + buf * kStage;
    const uint8_t* bA = bB + BN * 128;
    i32x8 aop[SM];
#pragma unroll
    for (int j = 0; j < SM; ++j) aop[j] = lds_operand(bA, wm * TM + 16 * j + rsub, c0);
    float sab[SM];
#pragma unroll
    for (int j = 0; j < SM; ++j) sab[j] = saC[j] * sbC;
#pragma unroll
    for (int i = 0; i < SN; ++i) {
      const i32x8 bop = lds_operand(bB, wn * TN + 16 * i + rsub, c0);
#pragma unroll
      for (int j = 0; j < SM; ++j) {
        const f32x4 p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            bop, aop[j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(p[r], sab[j], acc[i][j][r]);
      }
    }

    if (more) {
      uint8_t* nb = smem + (buf ^ 1) * kStage;
#pragma unroll
      for (int s = 0; s < CB; ++s)
        if (ldsB[s] >= 0) *reinterpret_cast<uint4*>(nb + ldsB[s]) = stB[s];
#pragma unroll
      for (int s = 0; s < CA; ++s)
        if (ldsA[s] >= 0) *reinterpret_cast<uint4*>(nb + ldsA[s]) = stA[s];
    }
    __syncthreads();
    buf ^= 1;
  }

  using OT = typename OutT<OUT_DT>::T;
  OT* C = reinterpret_cast<OT*>(a.c);
  const bool vec_ok = a.vec_ok != 0;

  if constexpr (SPLIT) {
    // partial tile layout: [split][tile][wave][i][j][lane][4] floats
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const int64_t tiles = (int64_t)gridDim.x * gridDim.y;
    constexpr int kTileFloats = BN * BM;
    float* mine = a.ws + ((int64_t)z * tiles + tile) * kTileFloats + wave * (SN * SM * 256);
#pragma unroll
    for (int i = 0; i < SN; ++i)
#pragma unroll
      for (int j = 0; j < SM; ++j)
        *reinterpret_cast<f32x4*>(mine + ((i * SM + j) * 64 + lane) * 4) = acc[i][j];
    __threadfence();
    __syncthreads();
    __shared__ int s_last;
    if (tid == 0) {
      const int old = atomicAdd(a.counters + tile, 1);
      s_last = (old == a.split - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
#pragma unroll
    for (int i = 0; i < SN; ++i)
#pragma unroll
      for (int j = 0; j < SM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int zz = 0; zz < a.split; ++zz) {
      const float* part = a.ws + ((int64_t)zz * tiles + tile) * kTileFloats + wave * (SN * SM * 256);
#pragma unroll
      for (int i = 0; i < SN; ++i)
#pragma unroll
        for (int j = 0; j < SM; ++j) {
          const f32x4 v = __builtin_nontemporal_load(
              reinterpret_cast<const f32x4*>(part + ((i * SM + j) * 64 + lane) * 4));
          acc[i][j] += v;
        }
    }
    if (tid == 0) a.counters[tile] = 0;
  }

#pragma unroll
  for (int j = 0; j < SM; ++j) {
    const int m = m0 + wm * TM + 16 * j + rsub;
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < SN; ++i) {
      const int n = n0 + wn * TN + 16 * i + 4 * c0;
      OT* dst = C + (int64_t)m * N + n;
      if (vec_ok && n + 3 < N) {
        store4<OUT_DT>(dst, acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) store1<OUT_DT>(dst + r, acc[i][j][r]);
      }
    }
  }
}

// ---- kernel table -------------------------------------------------------------

using KernelFn = void (*)(GemmArgs);

struct CfgEntry {
  int bn, bm, wn, wm;
  const char* name;
  KernelFn fn[3][2];  // [out_dt][split]
};

#define INFEROP_GEMM_CFG(BN, BM, WN, WM, NAME)                                                 \
  {BN, BM, WN, WM, NAME,                                                                       \
   {{gemm_kernel<BN, BM, WN, WM, kFp32, false>, gemm_kernel<BN, BM, WN, WM, kFp32, true>},     \
    {gemm_kernel<BN, BM, WN, WM, kFp16, false>, gemm_kernel<BN, BM, WN, WM, kFp16, true>},     \
    {gemm_kernel<BN, BM, WN, WM, kBf16, false>, gemm_kernel<BN, BM, WN, WM, kBf16, true>}}}

const CfgEntry kCfgs[] = {
    INFEROP_GEMM_CFG(128, 128, 2, 2, "n128_m128_w2x2"),
    INFEROP_GEMM_CFG(64, 16, 4, 1, "n64_m16_w4x1"),
    INFEROP_GEMM_CFG(64, 32, 4, 1, "n64_m32_w4x1"),
    INFEROP_GEMM_CFG(64, 64, 4, 1, "n64_m64_w4x1"),
    INFEROP_GEMM_CFG(256, 128, 2, 2, "n256_m128_w2x2"),
    INFEROP_GEMM_CFG(128, 256, 2, 2, "n128_m256_w2x2"),
};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

// ---- split-K workspace, one per (device, stream) ------------------------------

__global__ void fill_zero_kernel(int* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

struct Workspace {
  float* partials = nullptr;
  size_t partial_bytes = 0;
  int* counters = nullptr;
  size_t counter_count = 0;
};

std::mutex g_ws_mutex;
std::unordered_map<uint64_t, Workspace> g_ws;

hipError_t get_workspace(hipStream_t st, size_t partial_bytes, size_t counters, float** ws,
                         int** cnt) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t key = (uint64_t)(uintptr_t)st * 64u + (uint64_t)dev;
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Workspace& w = g_ws[key];
  if (w.partial_bytes < partial_bytes) {
    if (w.partials) {
      e = hipStreamSynchronize(st);
      if (e != hipSuccess) return e;
      (void)hipFree(w.partials);
      w.partials = nullptr;
      w.partial_bytes = 0;
    }
    const size_t bytes = partial_bytes + partial_bytes / 2;
    e = hipMalloc(&w.partials, bytes);
    if (e != hipSuccess) return e;
    w.partial_bytes = bytes;
  }
  if (w.counter_count < counters) {
    if (w.counters) {
      e = hipStreamSynchronize(st);
      if (e != hipSuccess) return e;
      (void)hipFree(w.counters);
      w.counters = nullptr;
      w.counter_count = 0;
    }
    const size_t count = counters < 4096 ? 4096 : counters * 2;
    e = hipMalloc(&w.counters, count * sizeof(int));
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st,
                       w.counters, (int64_t)count);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    w.counter_count = count;
  }
  *ws = w.partials;
  *cnt = w.counters;
  return hipSuccess;
}

int dt_index(int32_t out_dt) {
  switch (out_dt) {
    case kFp32: return 0;
    case kFp16: return 1;
    case kBf16: return 2;
    default: return -1;
  }
}

}  // namespace
}  // namespace inferop_hip

using namespace inferop_hip;

extern "C" int inferop_hip_gemm_num_configs(void) { return kNumCfgs; }

extern "C" int inferop_hip_gemm_config_info(int32_t cfg, inferop_gemm_cfg_info* info) {
  if (cfg < 0 || cfg >= kNumCfgs || !info) return hipErrorInvalidValue;
  info->bn = kCfgs[cfg].bn;
  info->bm = kCfgs[cfg].bm;
  info->waves = kCfgs[cfg].wn * kCfgs[cfg].wm;
  info->kind = 0;
  info->name = kCfgs[cfg].name;
  return hipSuccess;
}

extern "C" int inferop_hip_gemm_w8a8_block(void* c, const uint8_t* a_q, const float* a_scales,
                                           const uint8_t* b_q, const float* b_scales, int64_t m,
                                           int64_t n, int64_t k, int32_t out_dt,
                                           const inferop_gemm_launch* launch, void* stream) {
  const int di = dt_index(out_dt);
  if (di < 0 || !launch || launch->cfg < 0 || launch->cfg >= kNumCfgs) return hipErrorInvalidValue;
  if (m <= 0 || n <= 0 || k <= 0 || k % 128 != 0) return hipErrorInvalidValue;
  if (m > 0x7FFFFFFF || n > 0x7FFFFFFF || k > 0x7FFFFFFF) return hipErrorInvalidValue;
  const CfgEntry& cf = kCfgs[launch->cfg];
  const int kg = (int)(k / 128);
  int split = launch->split_k < 1 ? 1 : launch->split_k;
  if (split > kg) split = kg;
  const int64_t tn = (n + cf.bn - 1) / cf.bn;
  const int64_t tm = (m + cf.bm - 1) / cf.bm;
  if (tn > 0x7FFFFFFF || tm > 65535 || split > 65535) return hipErrorInvalidConfiguration;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int out_bytes = out_dt == kFp32 ? 4 : 2;
  const int vec_ok = (n % 4 == 0) && ((uintptr_t)c % (size_t)(4 * out_bytes) == 0);
  GemmArgs args{c,       a_q,    a_scales, b_q,    b_scales, nullptr,
                nullptr, (int)m, (int)n,   (int)k, split,    vec_ok};
  if (split > 1) {
    const size_t tiles = (size_t)(tn * tm);
    const size_t bytes = (size_t)split * tiles * (size_t)cf.bn * (size_t)cf.bm * sizeof(float);
    hipError_t e = get_workspace(st, bytes, tiles, &args.ws, &args.counters);
    if (e != hipSuccess) return e;
  }
  const dim3 grid((unsigned)tn, (unsigned)tm, (unsigned)split);
  const dim3 block(64 * cf.wn * cf.wm);
  hipLaunchKernelGGL(cf.fn[di][split > 1 ? 1 : 0], grid, block, 0, st, args);
  return hipGetLastError();
}
