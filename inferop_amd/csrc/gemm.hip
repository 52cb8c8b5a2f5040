// W8A8 blockwise-FP8 GEMM for gfx950 (CDNA4).
//
//   C[m,n] = sum_g sa[m,g] * sb[n/128,g] * sum_{k in group g} A[m,k] * B[n,k]
//   A: [M,K] E4M3, sa: [M,K/128] fp32, B: [N,K] E4M3, sb: [ceil(N/128),K/128] fp32
//
// Matrix cores: v_mfma_scale_f32_16x16x128_f8f6f4 with both formats E4M3 and
// unit E8M0 scales.  One instruction multiplies a 16x128 weight slice by a
// 16x128 activation slice -- exactly one 128-wide scale group -- so each MFMA
// yields the group's partial dot products, and the fp32 block scales are
// applied in VALU registers:  acc = fma(partial, sa[m,g] * sb[n/128,g], acc).
// The weight slice is the MFMA "A" operand and the activation slice the "B"
// operand, so a lane's four accumulator registers are four consecutive n of
// one output row m: one activation scale per lane per 16-row slice, one weight
// scale per wave (a wave never straddles a 128-row weight block, the scale
// sits in an SGPR), and the four values are contiguous in C.
//
// Operand layout: lane l supplies row (l % 16) of its 16-row slice and the
// 16-byte chunks (l / 16) and (l / 16 + 4) of the 128-byte group.  Both
// operands use the same chunk order, so the K permutation cancels.
//
// Three kernel families:
//
// * decode (M <= 64 per tile, HBM-bound): no barrier in the main loop.  Each
//   wave streams its 16 weight rows, U scale groups at a time, with direct
//   global->LDS loads into an LDS region only it uses (whole 128-byte rows per
//   8 lanes, the access pattern HBM streams best), reads them back in MFMA
//   layout, and takes the small activation tile from L2 straight into
//   registers.  The waves of a workgroup split the workgroup's K range and are
//   summed through LDS; workgroups split K further (split-K) and the last one
//   to finish a tile adds the partials in split order (deterministic).
//   Partials travel through device-coherent stores and loads and a
//   device-scope atomic counter, so no L2 writeback or invalidate is needed.
//
// * prefill (large M, MFMA-bound): a BN x BM output tile per workgroup, A and
//   B staged in LDS by direct global->LDS loads (global_load_lds_dwordx4, no
//   VGPR round trip), double-buffered so group g+1 streams in while group g is
//   multiplied.  LDS rows are 128 bytes = eight 16-byte chunks stored at
//   chunk ^ (row & 7): the eight lanes of a ds_read_b128 phase hit eight
//   different bank groups.  Tiles are renumbered so each XCD works on a
//   contiguous, M-grouped range of tiles (L2 reuse of A and B).
//
// * persistent prefill (large M, whole tiles): the same stage layout and
//   MFMA core in one workgroup per CU that walks its tiles without stopping
//   the pipeline between them; half the waves issue the stage loads and the
//   other half the output stores, so the stores of one tile drain while the
//   next is multiplied.
#include <atomic>
#include <mutex>
#include <type_traits>
#include <unordered_map>

#include "device_common.h"
#include "hip_launch.h"
#include "quant_group.h"

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
  int vec_ok;  // C rows can take 4-element vector stores (N % 4 == 0, C aligned)
  // grouped (MoE expert) GEMM; B and its scales hold `experts` matrices.
  // Contiguous layout (max_m == 0): A's rows sorted by expert, expert e owning
  // rows [offsets[e], offsets[e+1]).  Masked layout (max_m > 0): expert e
  // owns rows [e * max_m, e * max_m + offsets[e]) (offsets = valid counts).
  const int* offsets;
  int experts;
  int max_m;
  // persistent kernels (plain GEMM): the tiles of the last, partial round are
  // each cut into tail_split K ranges (1: whole tiles); their fp32 partials go
  // to ws and a second kernel adds them
  int tail_split;
};

// Raw buffer resource over `bytes` bytes at base (stride 0; dword3 selects a
// 32-bit data format so untyped loads are valid).  Loads at offsets >= bytes
// return zeros, which is how tiles past the last row of A or B are padded.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// 16 bytes per lane from the buffer at voffset + soffset into LDS at
// lds + 16 * lane (the LDS address is wave-uniform).
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t r, void* lds, int voffset,
                                                int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                           voffset, soffset, 0, 0);
}

// Direct-to-LDS loads as inline assembly, for kernels that wait for them
// explicitly (stage barriers, counted vmcnt waits): the compiler's wait analysis does not see
// these loads, so it never puts its own vmcnt waits in front of LDS reads or
// barriers on their account (it does wherever its LDS alias information is
// incomplete, and on a wave with global stores in flight such a wait would
// stall on the stores).  M0 carries the wave's LDS destination.  The compiler
// does not resolve hazards for inline assembly, so each load starts with five
// wait states: enough for an SGPR operand (buffer resource or offset) written
// by a VALU instruction such as v_readfirstlane, and for the M0 write ahead of
// an LDS DMA.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void asm_buffer_to_lds16(const u32x4& rsrc, uint32_t lds, int voffset,
                                                    int soffset) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(soffset), "{m0}"(lds)
               : "memory");
}
// Same with the non-temporal hint: for data read exactly once (streamed
// weights), so it does not push data that is read again out of the L2.
__device__ __forceinline__ void asm_buffer_to_lds16_nt(const u32x4& rsrc, uint32_t lds,
                                                       int voffset, int soffset) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen nt lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(soffset), "{m0}"(lds)
               : "memory");
}
__device__ __forceinline__ void asm_global_to_lds4(const void* p, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, off" : : "v"(p), "{m0}"(lds) : "memory");
}
// Raw buffer resource words (the fields make_rsrc sets) in SGPRs, for the
// inline-assembly loads.
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b),
               (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)),
               (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes), 0x00020000u};
}

// s_waitcnt immediate (gfx9 encoding): at most n vector memory operations of
// this wave outstanding and every LDS/scalar access completed.
__device__ constexpr int vmcnt_lgkm0_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

__device__ __forceinline__ f32x4 mfma_group(const i32x8& w, const i32x8& x) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, x, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0,
                                                          0, 127, 0, 127);
}

__device__ __forceinline__ i32x8 cat8(const u32x4& lo, const u32x4& hi) {
  return i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
               (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

// 32 operand bytes of one lane straight from global memory: chunks c0 and c0+4
// of the 128-byte group at p (p already points at chunk c0).
template <bool NT>
__device__ __forceinline__ i32x8 load_operand(const uint8_t* p) {
  const u32x4* q = reinterpret_cast<const u32x4*>(p);
  if constexpr (NT) {
    return cat8(__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 4));
  } else {
    return cat8(q[0], q[4]);
  }
}

__device__ __forceinline__ i32x8 lds_operand(const uint8_t* base, int row, int c0) {
  const uint8_t* r = base + row * 128;
  const int x = row & 7;
  const u32x4 lo = *reinterpret_cast<const u32x4*>(r + ((c0 ^ x) << 4));
  const u32x4 hi = *reinterpret_cast<const u32x4*>(r + ((c0 ^ x ^ 4) << 4));
  return cat8(lo, hi);
}

// Store a lane's 4 consecutive outputs of row m starting at column n.
template <int OUT_DT>
__device__ __forceinline__ void store_out4(const GemmArgs& a, int m, int n, const f32x4& v) {
  using OT = typename OutT<OUT_DT>::T;
  if (m >= a.m) return;
  OT* dst = reinterpret_cast<OT*>(a.c) + (int64_t)m * a.n + n;
  if (a.vec_ok && n + 3 < a.n) {
    store4<OUT_DT>(dst, v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (n + r < a.n) store1<OUT_DT>(dst + r, v[r]);
  }
}

// ---- split-K fixup -------------------------------------------------------------
// Called by every thread of a workgroup once its share of the tile partial is
// complete: this wave holds LP pairs (an f32x4 per lane each) that are pairs
// pair_base .. pair_base+LP-1 of the tile's `pairs` pairs; valid(q) says
// whether this lane's q-th pair carries data (inside M, owned by this wave).
// Returns true in the workgroup that arrives last for the tile; `part` then
// holds the sum over all splits, added in split order.  A lane's pair q sits
// at bytes (q * 64 + lane) * 16 of the wave's slot, so every store and load
// instruction moves 1 KB of contiguous memory.
//
// The partials are written and read with the sc1 cache policy (agent scope:
// past the CU's L1 and the XCD's non-coherent L2), as plain buffer accesses
// rather than atomic ones: the compiler serializes atomic loads (a full
// vmcnt(0) wait after each), which made the last workgroup's reads one round
// trip per split and per register -- M=1, N=2112, K=7168 with split 2 cost
// 12.5 us against 6.8 us unsplit.  Plain loads of all splits are issued
// together and waited for once.
constexpr int kSc1 = 16;  // buffer cache policy bit: sc1

template <int LP, typename Valid>
__device__ __forceinline__ bool splitk_fixup(const GemmArgs& a, f32x4 (&part)[LP], int split,
                                             int z, int tile, int64_t tiles, int pairs,
                                             int pair_base, int lane, Valid valid) {
  __shared__ int s_last;
  const __amdgpu_buffer_rsrc_t ws = make_rsrc(a.ws, (uint32_t)INFEROP_SPLITK_WS_BYTES);
  // byte offsets: the host keeps split * tiles * pairs * 1 KB within the workspace
  const int tile_bytes = pairs * 1024;
  const int split_bytes = (int)(tiles * tile_bytes);
  const int mine = z * split_bytes + tile * tile_bytes + pair_base * 1024 + lane * 16;
#pragma unroll
  for (int q = 0; q < LP; ++q) {
    if (!valid(q)) continue;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, part[q]), ws, mine + q * 1024,
                                           0, kSc1);
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores are acknowledged
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(a.counters + tile, 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    s_last = (old == split - 1);
  }
  __syncthreads();
  if (!s_last) return false;
  const int base = tile * tile_bytes + pair_base * 1024 + lane * 16;
  auto load = [&](int zz, int q) {
    return __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(ws, base + zz * split_bytes + q * 1024, 0, kSc1));
  };
  if constexpr (LP > 8) {
    // large tiles (never split by the automatic choice): one pair at a time,
    // which keeps the kernel's register budget
#pragma unroll
    for (int q = 0; q < LP; ++q) {
      if (!valid(q)) continue;
      f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int zz = 0; zz < split; ++zz) sum += load(zz, q);
      part[q] = sum;
    }
  } else {
    // The partials of ZB splits for QB pairs are loaded together before any
    // is added, so the loads travel in parallel rather than one split at a
    // time; each element still adds the splits in order 0, 1, ..., split - 1.
    // No load is issued past the last split.  The batch loops run their full
    // constant trip count with the split bound as a predicate (split is
    // uniform: a scalar branch), not as a `break`: a loop with an exit cannot
    // be unrolled, and the batch v[][] indexed by a loop variable would then
    // live in scratch memory rather than registers.
    constexpr int QB = LP < 4 ? LP : 4;
    constexpr int ZB = (LP <= 2 ? 16 : 8) / QB;
    static_assert(LP % QB == 0, "pairs in whole batches");
#pragma unroll
    for (int q0 = 0; q0 < LP; q0 += QB) {
      f32x4 sum[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sum[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int z0 = 0; z0 < split; z0 += ZB) {
        f32x4 v[ZB][QB];
#pragma unroll
        for (int zb = 0; zb < ZB; ++zb) {
          const bool live = z0 + zb < split;
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
            if (live && valid(q0 + qb)) v[zb][qb] = load(z0 + zb, q0 + qb);
        }
#pragma unroll
        for (int zb = 0; zb < ZB; ++zb) {
          const bool live = z0 + zb < split;
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
            if (live && valid(q0 + qb)) sum[qb] += v[zb][qb];
        }
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        if (valid(q0 + qb)) part[q0 + qb] = sum[qb];
    }
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(a.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// ---- decode kernel ---------------------------------------------------------------
// grid: x = N tiles of 16 rows, y = K splits, z = M tiles of 16*MT rows.
// The WK waves of a workgroup split the workgroup's scale groups.  A wave
// streams its 16 weight rows for up to U groups at a time with direct
// global->LDS loads into its own LDS region -- each load instruction reads 8
// whole 128-byte rows, the contiguous pattern HBM streams best -- while the
// activation slices come from L2 straight into registers; then it reads the
// weight operands back in MFMA layout (no barrier: the region is private).
// The WK slices are summed through LDS; K splits across workgroups go
// through the split-K fixup.
template <int MT, int WK, int U, int OUT_DT>
__global__ __launch_bounds__(64 * WK) void gemm_decode_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t bst[WK][U][2048];
  const int lane = threadIdx.x & 63;
  const int wk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int M = a.m, N = a.n, K = a.k;
  const int KG = K >> 7;
  const int NB = (N + 127) >> 7;
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.z * (16 * MT);
  const int split = gridDim.y, z = blockIdx.y;
  const int gz0 = (int)((int64_t)z * KG / split), gz1 = (int)((int64_t)(z + 1) * KG / split);
  const int cnt = gz1 - gz0;
  const int gw0 = gz0 + wk * cnt / WK, gw1 = gz0 + (wk + 1) * cnt / WK;
  const int rsub = lane & 15, c0 = lane >> 4;

  // DMA slots: instruction i of a group covers rows 8i .. 8i+7; lane -> row
  // 8i + (lane >> 3), 16-byte chunk (lane & 7) ^ (lane >> 3)
  const int lrow = lane >> 3;
  const int lcol = ((lane & 7) ^ lrow) * 16;
  const uint8_t* tileB = a.bq + (int64_t)n0 * K;
  const int nlast = N - 1 - n0;
  const int off0 = min(lrow, nlast) * K + lcol;
  const int off1 = min(8 + lrow, nlast) * K + lcol;
  const float* sbp = a.bs + (int64_t)min(n0 >> 7, NB - 1) * KG;
  const uint8_t* ap[MT];
  const float* sap[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    const int row = min(m0 + 16 * j + rsub, M - 1);
    ap[j] = a.aq + (int64_t)row * K + c0 * 16;
    sap[j] = a.as + (int64_t)row * KG;
  }

  f32x4 acc[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int g = gw0; g < gw1; g += U) {
    i32x8 av[U][MT];
    float sav[U][MT], sbv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int gg = min(g + u, gw1 - 1);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(tileB + (off0 + gg * 128)),
          (__attribute__((address_space(3))) void*)(&bst[wk][u][0]), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(tileB + (off1 + gg * 128)),
          (__attribute__((address_space(3))) void*)(&bst[wk][u][1024]), 16, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int gg = min(g + u, gw1 - 1);
#pragma unroll
      for (int j = 0; j < MT; ++j) av[u][j] = load_operand<false>(ap[j] + gg * 128);
#pragma unroll
      for (int j = 0; j < MT; ++j) sav[u][j] = sap[j][gg];
      sbv[u] = sbp[gg];
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's rows are in its LDS region
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (g + u < gw1) {
        const i32x8 bv = lds_operand(&bst[wk][u][0], rsub, c0);
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const f32x4 pv = mfma_group(bv, av[u][j]);
          const float s = sav[u][j] * sbv[u];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[j][r] = __builtin_fmaf(pv[r], s, acc[j][r]);
        }
      }
    }
  }

  // sum the WK slices through LDS: wave 0 ends up with the tile
  if constexpr (WK > 1) {
    __shared__ f32x4 red[WK - 1][MT][64];
    if (wk > 0) {
#pragma unroll
      for (int j = 0; j < MT; ++j) red[wk - 1][j][lane] = acc[j];
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int w = 0; w < WK - 1; ++w)
#pragma unroll
        for (int j = 0; j < MT; ++j) acc[j] += red[w][j][lane];
    }
  }

  if (split > 1) {
    const int tile = blockIdx.z * gridDim.x + blockIdx.x;
    const int64_t tiles = (int64_t)gridDim.x * gridDim.z;
    auto valid = [&](int q) { return wk == 0 && m0 + 16 * q + rsub < M; };
    if (!splitk_fixup<MT>(a, acc, split, z, tile, tiles, MT, 0, lane, valid)) return;
  }
  if (wk == 0) {
#pragma unroll
    for (int j = 0; j < MT; ++j) store_out4<OUT_DT>(a, m0 + 16 * j + rsub, n0 + 4 * c0, acc[j]);
  }
}

// ---- decode kernel with LDS-staged activations ------------------------------------
// grid: x = N tiles of 16 rows, y = K splits, z = M tiles of 16 rows.
// As gemm_decode_kernel<1, ...>, but the activation slice of every scale group
// also arrives by direct-to-LDS loads (8 lanes per 128-byte row segment, the
// pattern the weights use) instead of 16-byte register loads that touch half
// lines, and the U groups of a batch are consumed in the order they land.
// Each slot is its own LDS variable, so the compiler waits for exactly the
// loads of the slot being read rather than for the whole batch.
template <int WK, int U, int OUT_DT>
__global__ __launch_bounds__(64 * WK) void gemm_decode_lds_kernel(GemmArgs a) {
  static_assert(U >= 1 && U <= 4, "1 to 4 slots per wave");
  constexpr int kSlot = WK * 4096;  // per wave: 16 weight rows + 16 activation rows
  __shared__ __attribute__((aligned(1024))) uint8_t slot0[kSlot];
  __shared__ __attribute__((aligned(1024))) uint8_t slot1[U > 1 ? kSlot : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t slot2[U > 2 ? kSlot : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t slot3[U > 3 ? kSlot : 16];
  auto slot = [&](int u) -> uint8_t* {
    return u == 0 ? slot0 : u == 1 ? slot1 : u == 2 ? slot2 : slot3;
  };
  const int lane = threadIdx.x & 63;
  const int wk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int M = a.m, N = a.n, K = a.k;
  const int KG = K >> 7;
  const int NB = (N + 127) >> 7;
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.z * 16;
  const int split = gridDim.y, z = blockIdx.y;
  const int gz0 = (int)((int64_t)z * KG / split), gz1 = (int)((int64_t)(z + 1) * KG / split);
  const int cnt = gz1 - gz0;
  const int gw0 = gz0 + wk * cnt / WK, gw1 = gz0 + (wk + 1) * cnt / WK;
  const int rsub = lane & 15, c0 = lane >> 4;
  // DMA slots: instruction h covers rows 8h .. 8h+7; lane -> row 8h + (lane >> 3),
  // chunk (lane & 7) ^ (lane >> 3).  Rows past the end read as zeros.
  const int lrow = lane >> 3;
  const int lcol = ((lane & 7) ^ lrow) * 16;
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(a.bq + (int64_t)n0 * K, (uint32_t)(min(16, N - n0) * K));
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(a.aq + (int64_t)m0 * K, (uint32_t)(min(16, M - m0) * K));
  const int off0 = lrow * K + lcol, off1 = (8 + lrow) * K + lcol;
  const float* sbp = a.bs + (int64_t)min(n0 >> 7, NB - 1) * KG;
  const float* sap = a.as + (int64_t)min(m0 + rsub, M - 1) * KG;
  const int wo = wk * 4096;  // this wave's part of every slot

  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int g = gw0; g < gw1; g += U) {
    // scales first, then the slots in the order they are consumed
    float sav[U], sbv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int gg = min(g + u, gw1 - 1);
      sav[u] = sap[gg];
      sbv[u] = sbp[gg];
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int gg = min(g + u, gw1 - 1);
      uint8_t* sl = slot(u) + wo;
      buffer_to_lds16(rB, sl, off0, gg * 128);
      buffer_to_lds16(rB, sl + 1024, off1, gg * 128);
      buffer_to_lds16(rA, sl + 2048, off0, gg * 128);
      buffer_to_lds16(rA, sl + 3072, off1, gg * 128);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (g + u < gw1) {
        const uint8_t* sl = slot(u) + wo;
        const f32x4 pv = mfma_group(lds_operand(sl, rsub, c0), lds_operand(sl + 2048, rsub, c0));
        const float sc = sav[u] * sbv[u];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = __builtin_fmaf(pv[r], sc, acc[r]);
      }
    }
  }

  // sum the WK slices through LDS: wave 0 ends up with the tile
  if constexpr (WK > 1) {
    __shared__ f32x4 red[WK - 1][64];
    if (wk > 0) red[wk - 1][lane] = acc;
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int w = 0; w < WK - 1; ++w) acc += red[w][lane];
    }
  }
  f32x4 part[1] = {acc};
  if (split > 1) {
    const int tile = blockIdx.z * gridDim.x + blockIdx.x;
    const int64_t tiles = (int64_t)gridDim.x * gridDim.z;
    auto valid = [&](int) { return wk == 0 && m0 + rsub < M; };
    if (!splitk_fixup<1>(a, part, split, z, tile, tiles, 1, 0, lane, valid)) return;
  }
  if (wk == 0) store_out4<OUT_DT>(a, m0 + rsub, n0 + 4 * c0, part[0]);
}

// ---- decode kernel for several activation tiles per weight stripe -------------------
// grid: x = N stripes of 16 weight rows, y = M tiles of 16*MT rows.
// A workgroup owns one 16-row weight stripe over the whole K range and MT
// 16-row activation tiles; its WK waves split the scale groups and are summed
// through LDS at the end (no split-K, so no round trip through device-coherent
// partials).  Each weight byte leaves HBM once (non-temporal loads, so the
// stream does not evict the activations); the activations, shared by every
// stripe, come from L2.  A wave streams its groups through two private rings:
// UW weight slots (2 KB each), refilled UW groups ahead, and UA activation
// slots (MT tiles), refilled UA groups ahead.  The loads are inline assembly
// issued in a fixed pattern, so a single constant vmcnt wait covers the next
// group in every iteration; past the wave's last group the pattern continues
// with 4-byte loads of a weight scale (kept only for the count).
//
// Scales: with PRE, a wave loads the activation scales of its MT tiles and the
// weight scales for all its groups into LDS once, before the rings start, as
// row-contiguous runs (a per-group load of 16*MT activation scales touches
// 16*MT cache lines, more than the weight slice itself).  That needs at most
// wide_scale_cap() groups per wave; longer ranges use the kernel without
// PRE, whose activation slots also carry that group's scales.  The cap keeps
// the configurations small enough for two workgroups per CU (LDS), which is
// worth more than preloading for longer K.
__host__ __device__ constexpr int wide_scale_cap() { return 16; }

// Grouped mode (GROUPED): grid y enumerates virtual M tiles of 16*MT rows as in
// the tiled kernel's grouped mode (grouped_tile); a workgroup streams one
// 16-row stripe of its expert's weights against that expert's rows.
//
// NT > 1: a workgroup owns NT adjacent stripes (16 * NT weight rows inside one
// 128-row weight block) and every wave multiplies each activation slice with
// all NT weight slices, so a CU reads the activations once per 16 * NT weight
// rows instead of once per 16.  With fewer stripes than CUs left, the K range
// is split across workgroups (grid z) and the partials meet in the split-K
// fixup.
//
// AR = 8 (one activation tile, M <= 8 rows per workgroup): a tile is 8 rows,
// one load per group instead of two; the MFMA's other 8 columns read stale
// LDS and their outputs are never stored or summed into stored outputs (each
// output column of the MFMA depends only on its own activation row).
template <int MT, int WK, int UW, int UA, bool PRE, int OUT_DT, bool GROUPED = false, int NT = 1,
          int AR = 16>
__global__ __launch_bounds__(64 * WK) void gemm_decode_wide_kernel(GemmArgs a) {
  static_assert(NT == 1 || NT == 2 || NT == 4 || NT == 8, "stripes inside one weight block");
  static_assert(NT == 1 || !GROUPED, "grouped mode streams one stripe");
  static_assert(AR == 16 || (AR == 8 && MT == 1 && !GROUPED), "8-row tiles: one plain tile");
  constexpr int kW = NT * 2048;                       // 16 * NT weight rows x 128 B
  constexpr int kCap = wide_scale_cap();
  constexpr int kOffSa = MT * AR * 128;               // in an activation slot (no PRE)
  constexpr int kOffSb = kOffSa + 256;
  constexpr int kA = MT * AR * 128 + (PRE ? 0 : 512); // MT tiles (+ 64 sa + 64 sb)
  constexpr int kSaF = PRE ? 16 * MT * kCap : 0;      // preloaded sa floats, [row][group]
  constexpr int kScale = PRE ? kSaF * 4 + 256 : 0;    // + up to 64 sb floats
  constexpr int kWave = UW * kW + UA * kA + kScale;
  constexpr int kPerIter = 2 * NT + (AR / 8) * MT + (PRE ? 0 : 2);  // loads issued per group
  constexpr int kPairs = NT * MT;                     // 16x16 output blocks
  constexpr int kLP = (kPairs + WK - 1) / WK;         // blocks per wave at the end
  constexpr int kWait = (UA - 1) * kPerIter;          // loads that may stay in flight
  static_assert(UW >= UA && UA >= 2 && kWait <= 63, "ring sizes");
  static_assert(MT >= 1 && MT <= 4 && kCap <= 64, "1 to 4 activation tiles");
  static_assert(kPairs * 1024 <= kWave, "the end-of-kernel sum fits in the slots");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[WK * kWave];

  const int lane = threadIdx.x & 63;
  const int wk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int M = a.m, N = a.n, K = a.k;
  const int KG = K >> 7;
  const int NB = (N + 127) >> 7;
  const int n0 = blockIdx.x * (16 * NT);
  // activation rows [m0, mend); the expert's weights and scales when grouped
  int m0, mend;
  const uint8_t* bq = a.bq;
  const float* bs = a.bs;
  if constexpr (GROUPED) {
    int e, r0, r1;
    if (!grouped_tile<16 * MT>(a, (int)blockIdx.y, lane, &e, &r0, &r1)) return;
    m0 = r0;
    mend = r1;
    bq += (int64_t)e * N * K;
    bs += (int64_t)e * NB * KG;
  } else {
    m0 = blockIdx.y * (AR * MT);
    mend = M;
  }
  // split z (grid z) covers the scale groups [gz0, gz1); the waves split those
  const int split = gridDim.z, z = blockIdx.z;
  const int gz0 = (int)((int64_t)z * KG / split), gz1 = (int)((int64_t)(z + 1) * KG / split);
  const int cz = gz1 - gz0;
  const int gw0 = gz0 + wk * cz / WK, gw1 = gz0 + (wk + 1) * cz / WK;
  const int cnt = gw1 - gw0;
  const int rsub = lane & 15, c0 = lane >> 4;
  const int arow = rsub % AR;  // activation slice row a lane reads (8-row tiles: again 0-7)
  const int lrow = lane >> 3;
  const int loff = lrow * K + ((lane & 7) ^ lrow) * 16;
  uint8_t* const wave_lds = smem + wk * kWave;
  const uint32_t wbase = lds_addr(wave_lds);
  const uint32_t abase = wbase + UW * kW;
  const uint32_t sbase = abase + UA * kA;
  const float* const sa_l = reinterpret_cast<const float*>(wave_lds + UW * kW + UA * kA);
  const float* const sb_l = sa_l + kSaF;

  f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (cnt > 0) {
    // rows past the end of A or B read as zeros
    const u32x4 rB = rsrc_words(bq + (int64_t)n0 * K, (uint32_t)(min(16 * NT, N - n0) * K));
    const u32x4 rA = rsrc_words(a.aq + (int64_t)m0 * K, (uint32_t)(min(AR * MT, mend - m0) * K));
    const float* sb_src = bs + (int64_t)min(n0 >> 7, NB - 1) * KG + gw0;
    const float* sa_src = a.as + (int64_t)(m0 + min(lane % (16 * MT), mend - 1 - m0)) * KG + gw0;
    if constexpr (PRE) {
      // entry (r, g) at float r * cnt + g: consecutive lanes read consecutive
      // groups of one activation row
      const int E = 16 * MT * cnt;
      for (int t = 0; t * 64 < E; ++t) {
        const int idx = min(t * 64 + lane, E - 1);
        const int r = idx / cnt, g = idx - r * cnt;
        asm_global_to_lds4(a.as + (int64_t)min(m0 + r, mend - 1) * KG + gw0 + g, sbase + t * 256);
      }
      asm_global_to_lds4(sb_src + min(lane, cnt - 1), sbase + kSaF * 4);
    }
    auto issue_w = [&](int i) {  // group gw0 + i into weight slot i % UW
      const uint32_t dst = wbase + (uint32_t)(i % UW) * kW;
      if (i >= cnt) {
#pragma unroll
        for (int h = 0; h < 2 * NT; ++h) asm_global_to_lds4(sb_src, dst);
        return;
      }
      const int g = gw0 + i;
#pragma unroll
      for (int h = 0; h < 2 * NT; ++h)
        asm_buffer_to_lds16_nt(rB, dst + h * 1024, loff, 8 * h * K + g * 128);
    };
    auto issue_a = [&](int i) {  // group gw0 + i into activation slot i % UA
      const uint32_t dst = abase + (uint32_t)(i % UA) * kA;
      if (i >= cnt) {
#pragma unroll
        for (int h = 0; h < kPerIter - 2 * NT; ++h) asm_global_to_lds4(sb_src, dst);
        return;
      }
      const int g = gw0 + i;
#pragma unroll
      for (int h = 0; h < (AR / 8) * MT; ++h)
        asm_buffer_to_lds16(rA, dst + h * 1024, loff, 8 * h * K + g * 128);
      if constexpr (!PRE) {
        asm_global_to_lds4(sa_src + i, dst + kOffSa);
        asm_global_to_lds4(sb_src + i, dst + kOffSb);
      }
    };
    // Prologue in the loop's issue pattern: the weight slots beyond the
    // activation depth first, then (weight, activation) pairs; after it, and
    // after every iteration, exactly kWait loads follow the activations of the
    // group consumed next (the scale preload comes before all of them).
    for (int s = 0; s < UW - UA; ++s) issue_w(s);
#pragma unroll
    for (int j = 0; j < UA; ++j) {
      issue_w(UW - UA + j);
      issue_a(j);
    }
    for (int i = 0; i < cnt; ++i) {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(kWait));  // group i has landed
      asm volatile("" ::: "memory");
      const uint8_t* W = wave_lds + (i % UW) * kW;
      const uint8_t* A = wave_lds + UW * kW + (i % UA) * kA;
      const float sb = PRE ? sb_l[i] : reinterpret_cast<const float*>(A + kOffSb)[0];
      if constexpr (NT == 1) {
        const i32x8 wop = lds_operand(W, rsub, c0);
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const f32x4 pv = mfma_group(wop, lds_operand(A + j * AR * 128, arow, c0));
          const float sa = PRE ? sa_l[(16 * j + rsub) * cnt + i]
                               : reinterpret_cast<const float*>(A + kOffSa)[16 * j + rsub];
          const float sc = sa * sb;
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[0][j][r] = __builtin_fmaf(pv[r], sc, acc[0][j][r]);
        }
      } else {
        // the MT activation slices once, then each weight slice against them
        i32x8 aop[MT];
        float sc[MT];
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          aop[j] = lds_operand(A + j * AR * 128, arow, c0);
          const float sa = PRE ? sa_l[(16 * j + rsub) * cnt + i]
                               : reinterpret_cast<const float*>(A + kOffSa)[16 * j + rsub];
          sc[j] = sa * sb;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const i32x8 wop = lds_operand(W + t * 2048, rsub, c0);
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            const f32x4 pv = mfma_group(wop, aop[j]);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[t][j][r] = __builtin_fmaf(pv[r], sc[j], acc[t][j][r]);
          }
        }
      }
      // the slots of group i are read (operands in registers) before refilling
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue_w(i + UW);
      issue_a(i + UA);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(0));  // tail loads have landed
  }

  // Output block p = t * MT + j (weight slice t, activation tile j).  The WK
  // slices are summed through LDS (the slots are free now) in wave order;
  // wave w then owns blocks [w * kLP, (w + 1) * kLP).
  f32x4 part[kLP];
  if constexpr (WK > 1) {
    __syncthreads();
    f32x4* red = reinterpret_cast<f32x4*>(smem);  // [WK][kPairs][64]
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < MT; ++j) red[(wk * kPairs + t * MT + j) * 64 + lane] = acc[t][j];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kLP; ++q) {
      const int p = wk * kLP + q;
      if (p >= kPairs) continue;
      f32x4 s = red[p * 64 + lane];
      for (int w = 1; w < WK; ++w) s += red[(w * kPairs + p) * 64 + lane];
      part[q] = s;
    }
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < MT; ++j) part[t * MT + j] = acc[t][j];
  }
  auto row_of = [&](int q) { return m0 + 16 * ((wk * kLP + q) % MT) + rsub; };
  const bool lane_row = AR == 16 || rsub < AR;  // with 8-row tiles, lanes of rows 8-15 hold no row
  if (split > 1) {
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const int64_t tiles = (int64_t)gridDim.x * gridDim.y;
    auto valid = [&](int q) { return wk * kLP + q < kPairs && lane_row && row_of(q) < mend; };
    if (!splitk_fixup<kLP>(a, part, split, z, tile, tiles, kPairs, wk * kLP, lane, valid)) return;
  }
#pragma unroll
  for (int q = 0; q < kLP; ++q) {
    const int p = wk * kLP + q;
    if (p < kPairs && lane_row && row_of(q) < mend)
      store_out4<OUT_DT>(a, row_of(q), n0 + 16 * (p / MT) + 4 * c0, part[q]);
  }
}

// ---- decode GEMM that quantizes its own activations --------------------------------
// quant_fp8_per_token_group (group 128) and the GEMM in one launch, for M <= 8.
// grid: x = N stripes of 16 weight rows.  As the wide decode kernel with one
// 8-row activation tile (AR = 8, NT = MT = 1, no K split): a workgroup owns
// one stripe over the whole K range and its WK waves split the scale groups.
// Each wave first issues its weight ring (UW groups, direct-to-LDS,
// non-temporal), then the loads of the activation rows of all its groups at
// once (so they cost one round trip, not one per group), then quantizes them
// with the quantizer's own per-group code (qgroup::quant_group_lane: one DPP
// row per (row, group), four per step, so the work is proportional to M)
// into a private LDS region in the layout the MFMA operand read expects
// (8 rows x 128 B per group, 16-byte chunks swizzled by row), with the
// scales beside it.  Every (row, group) is also written to q / qs by exactly
// one workgroup (the one whose index is the item's index modulo the grid), so
// q and qs equal the quantizer's output.  The main loop then streams the
// weights through the ring as the wide decode kernel does (one fixed load
// pattern, one constant vmcnt wait) and multiplies in the same order as the
// 8-row wide decode kernel, whose output it reproduces bit for bit.  Rows
// M..7 of the region are never written: their MFMA columns are never stored.
// The activations are quantized again by every workgroup (M x K elements
// each), which only pays for a few rows; the host sends larger M to the
// quantizer and the GEMM as two launches.
__host__ __device__ constexpr int quant_gemm_cap() { return 8; }  // groups per wave

template <int WK, int DT, int OUT_DT>
__global__ __launch_bounds__(64 * WK) void gemm_quant_decode_kernel(GemmArgs a, const void* x,
                                                                    uint8_t* q, float* qs) {
  constexpr int UW = 4;
  constexpr int kCap = quant_gemm_cap();
  constexpr int kSteps = 8 * kCap / 4;  // (row, group) items, four per step
  constexpr int kW = 2048;              // 16 weight rows x 128 B
  constexpr int kA = 1024;              // 8 activation rows x 128 B
  constexpr int kWave = UW * kW + kCap * kA + 8 * kCap * 4;
  constexpr int kPerIter = 2;                // loads issued per group
  constexpr int kWait = (UW - 1) * kPerIter;  // loads that may stay in flight
  static_assert(WK * 64 * 16 <= WK * kWave, "the end-of-kernel sum fits in the slots");
  using I = qgroup::In<DT>;
  constexpr int kWords = I::kWords;  // 32-bit words of a lane's 8 elements
  __shared__ __attribute__((aligned(1024))) uint8_t smem[WK * kWave];

  const int lane = threadIdx.x & 63;
  const int wk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int M = a.m, N = a.n, K = a.k;
  const int KG = K >> 7;
  const int NB = (N + 127) >> 7;
  const int n0 = blockIdx.x * 16;
  const int gw0 = wk * KG / WK, gw1 = (wk + 1) * KG / WK;
  const int cnt = gw1 - gw0;
  const int rsub = lane & 15, c0 = lane >> 4;
  const int arow = rsub & 7;  // activation row a lane's MFMA column reads
  const int lrow = lane >> 3;
  const int loff = lrow * K + ((lane & 7) ^ lrow) * 16;
  uint8_t* const wave_lds = smem + wk * kWave;
  const uint32_t wbase = lds_addr(wave_lds);
  uint8_t* const act = wave_lds + UW * kW;                        // [kCap][8][128]
  float* const sa_l = reinterpret_cast<float*>(act + kCap * kA);  // [8][kCap]

  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  if (cnt > 0) {
    const u32x4 rB = rsrc_words(a.bq + (int64_t)n0 * K, (uint32_t)(min(16, N - n0) * K));
    const float* sb_src = a.bs + (int64_t)min(n0 >> 7, NB - 1) * KG + gw0;
    auto issue_w = [&](int i) {  // group gw0 + i into weight slot i % UW
      const uint32_t dst = wbase + (uint32_t)(i % UW) * kW;
      if (i >= cnt) {
        // past the wave's last group: the same number of loads (of a weight
        // scale), so the constant wait below stays exact
#pragma unroll
        for (int h = 0; h < 2; ++h) asm_global_to_lds4(sb_src, dst);
        return;
      }
      const int g = gw0 + i;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        asm_buffer_to_lds16_nt(rB, dst + h * 1024, loff, 8 * h * K + g * 128);
    };
#pragma unroll
    for (int j = 0; j < UW; ++j) issue_w(j);

    // The wave's (row, group) items, four per step: every load first (the
    // steps are unrolled and predicated, so the values stay in registers and
    // the loads travel together), then the quantization.  Memory operations
    // complete in issue order, so the wait for these loads also covers the
    // ring's first groups, which the first multiply needs anyway.
    const float sbv = sb_src[min(lane, cnt - 1)];  // weight scale of group `lane`
    const int sub = lane & 15;
    const int items = M * cnt;
    const int steps = (items + 3) >> 2;
    uint32_t w[kSteps][kWords];
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      if (st < steps) {
        const int t = min(4 * st + (lane >> 4), items - 1);
        const int r = t / cnt, i = t - r * cnt;
        const int64_t e0 = (int64_t)r * K + (gw0 + i) * 128 + sub * 8;
        const u32x4* src = reinterpret_cast<const u32x4*>(
            reinterpret_cast<const uint8_t*>(x) + e0 * (DT == kFp32 ? 4 : 2));
#pragma unroll
        for (int v = 0; v < kWords / 4; ++v) {
          const u32x4 tv = src[v];
          w[st][4 * v + 0] = tv.x;
          w[st][4 * v + 1] = tv.y;
          w[st][4 * v + 2] = tv.z;
          w[st][4 * v + 3] = tv.w;
        }
      }
    }
    const int grid = (int)gridDim.x;
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      if (st < steps) {
        const int tl = 4 * st + (lane >> 4);
        const int t = min(tl, items - 1);  // every lane takes part in the row reduction
        const int r = t / cnt, i = t - r * cnt, g = gw0 + i;
        uint32_t lo, hi;
        float s;
        qgroup::quant_group_lane<DT>(w[st], lo, hi, s);
        if (tl < items) {
          // bytes [8 sub, 8 sub + 8) of the row: half (sub & 1) of chunk sub / 2
          *reinterpret_cast<u32x2*>(act + i * kA + r * 128 +
                                    ((((sub >> 1) ^ (r & 7)) << 4) | ((sub & 1) << 3))) =
              u32x2{lo, hi};
          if (sub == 0) sa_l[r * kCap + i] = s;
          if ((r * KG + g) % grid == (int)blockIdx.x) {
            *reinterpret_cast<u32x2*>(q + (int64_t)r * K + g * 128 + sub * 8) = u32x2{lo, hi};
            if (sub == 0) qs[(int64_t)r * KG + g] = s;
          }
        }
      }
    }

    for (int i = 0; i < cnt; ++i) {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(kWait));  // group i has landed
      asm volatile("" ::: "memory");
      const i32x8 wop = lds_operand(wave_lds + (i % UW) * kW, rsub, c0);
      const f32x4 pv = mfma_group(wop, lds_operand(act + i * kA, arow, c0));
      const float sb = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sbv), i));
      const float sc = sa_l[arow * kCap + i] * sb;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = __builtin_fmaf(pv[r], sc, acc[r]);
      // the slot of group i is read (operand in registers) before refilling
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue_w(i + UW);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(0));  // tail loads have landed
  }

  // the WK waves' tiles summed through LDS in wave order (as the wide kernel)
  if constexpr (WK > 1) {
    __syncthreads();
    f32x4* red = reinterpret_cast<f32x4*>(smem);  // [WK][64]
    red[wk * 64 + lane] = acc;
    __syncthreads();
    if (wk != 0) return;
    acc = red[lane];
    for (int w = 1; w < WK; ++w) acc += red[w * 64 + lane];
  }
  if (rsub < 8 && rsub < M) store_out4<OUT_DT>(a, rsub, n0 + 4 * c0, acc);
}

// ---- prefill kernel --------------------------------------------------------------
// grid (tiles, K splits); waves arranged WN (along N) x WM (along M).

// The hardware deals workgroups to the 8 XCDs round-robin in linear launch
// order.  Renumber linear id b of nblk so that each XCD owns a contiguous
// range of logical ids (a bijection on [0, nblk) for any nblk): XCD x holds
// nblk / 8 ids, plus one when x < nblk % 8.
__device__ __forceinline__ int xcd_contiguous(int b, int nblk) {
  const int q = nblk >> 3, r = nblk & 7, x = b & 7;
  return x * q + min(x, r) + (b >> 3);
}

__device__ __forceinline__ void tile_of(int id, int tiles_n, int tiles_m, int* tn, int* tm) {
  // Groups of GM tile-rows along M walk across all N tiles: the A rows of a
  // group and the B rows of the current column stay hot in L2.
  constexpr int GM = 8;
  const int per_group = GM * tiles_n;
  const int grp = id / per_group;
  const int first_m = grp * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int in_grp = id - grp * per_group;
  *tm = first_m + in_grp % gm;
  *tn = in_grp / gm;
}

// Workgroup barrier for the LDS pipeline: wait until this wave's stage loads
// (all but the newest n vector memory operations) have landed in LDS and its
// LDS reads are done, then s_barrier.  Unlike __syncthreads() it does not
// wait for every outstanding global load, so later stages stay in flight.
// The empty asm statements keep the compiler from moving memory accesses
// across the barrier.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(N));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Grouped mode (GROUPED): grid x enumerates (N tile, virtual M tile) with
// tiles_n * (ceil(M/BM) + experts) entries, enough for every expert's
// ceil(rows/BM) M tiles.  A workgroup finds its expert by a prefix sum of the
// experts' tile counts (read from the device offsets or counts, clamped so
// that any values stay in bounds: offsets to [0, M], counts to [0, max_m]) and
// exits if its virtual tile is past the last one.
// Its rows are the expert's [r0, r1) slice of that tile; B and the weight
// scales are the expert's; rows past r1 read as zeros and are not stored.
template <int BM>
__device__ __forceinline__ bool grouped_tile(const GemmArgs& a, int tmv, int lane, int* e_out,
                                             int* r0_out, int* r1_out) {
  const int M = a.m, E = a.experts;
  int cum = 0;
  for (int c0 = 0; c0 < E; c0 += 64) {
    const int ei = c0 + lane;
    int lo = 0, hi = 0, cnt = 0;
    if (ei < E) {
      if (a.max_m > 0) {
        lo = ei * a.max_m;
        hi = lo + min(max(a.offsets[ei], 0), a.max_m);
      } else {
        lo = min(max(a.offsets[ei], 0), M);
        hi = min(max(a.offsets[ei + 1], lo), M);
      }
      cnt = (hi - lo + BM - 1) / BM;
    }
    int incl = cnt;  // inclusive prefix sum over the wave's 64 experts
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d);
      if (lane >= d) incl += v;
    }
    const int total = __shfl(incl, 63);
    if (tmv < cum + total) {
      const unsigned long long hit = __ballot(cum + incl > tmv);
      const int l = __builtin_ctzll(hit);
      const int before = cum + __shfl(incl - cnt, l);
      const int r0 = __shfl(lo, l) + (tmv - before) * BM;
      *e_out = __builtin_amdgcn_readfirstlane(c0 + l);
      *r0_out = __builtin_amdgcn_readfirstlane(r0);
      *r1_out = __builtin_amdgcn_readfirstlane(min(r0 + BM, __shfl(hi, l)));
      return true;
    }
    cum += total;
  }
  return false;
}

// Number of (expert, row block) M tiles: the sum of ceil(rows / BM) over the
// experts, rows as grouped_tile forms them.
template <int BM>
__device__ __forceinline__ int grouped_mtiles(const GemmArgs& a, int lane) {
  const int M = a.m, E = a.experts;
  int total = 0;
  for (int c0 = 0; c0 < E; c0 += 64) {
    const int ei = c0 + lane;
    int cnt = 0;
    if (ei < E) {
      int lo, hi;
      if (a.max_m > 0) {
        lo = ei * a.max_m;
        hi = lo + min(max(a.offsets[ei], 0), a.max_m);
      } else {
        lo = min(max(a.offsets[ei], 0), M);
        hi = min(max(a.offsets[ei + 1], lo), M);
      }
      cnt = (hi - lo + BM - 1) / BM;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) cnt += __shfl_xor(cnt, d);
    total += cnt;
  }
  return __builtin_amdgcn_readfirstlane(total);
}

template <int BN, int BM, int WN, int WM, int STAGES, int OUT_DT, bool GROUPED = false>
__global__ __launch_bounds__(64 * WN * WM) void gemm_prefill_kernel(GemmArgs a) {
  constexpr int NW = WN * WM;
  constexpr int TN = BN / WN, TM = BM / WM;
  constexpr int SN = TN / 16, SM = TM / 16;
  // one stage in LDS: B tile | A tile | activation scales | weight scale
  constexpr int kOffA = BN * 128;
  constexpr int kOffSA = (BN + BM) * 128;
  constexpr int kSaWaves = (BM + 63) / 64;  // waves that fetch activation scales
  constexpr int kOffSB = kOffSA + kSaWaves * 256;
  constexpr int kStage = ((kOffSB + 256) + 1023) / 1024 * 1024;
  constexpr int RB = BN / 8 / NW;  // 1 KB row blocks of B each wave loads per stage
  // A has BM / 8 row blocks; when there are fewer than waves, the extra waves
  // repeat a block (same bytes to the same LDS place) so that every wave
  // issues the same number of loads per stage, which the wait counts assume.
  constexpr int kABlocks = BM / 8;
  constexpr int RA = (kABlocks + NW - 1) / NW;
  constexpr int kLoadsPerStage = RB + RA + 1;  // + one scale load per wave
  constexpr int D = STAGES - 1;                // prefetch distance in scale groups
  static_assert(STAGES >= 2 && STAGES <= 4, "2 to 4 LDS stages");
  static_assert(TN % 16 == 0 && TM % 16 == 0, "wave tile must be a multiple of 16");
  static_assert(128 % TN == 0, "a wave must stay inside one 128-row weight block");
  static_assert(BN >= 128 ? BN % 128 == 0 : 128 % BN == 0, "tiles align to weight blocks");
  static_assert(BN % (8 * NW) == 0, "B row blocks must split evenly over the waves");
  static_assert((BM < 64 || BM % 64 == 0) && kSaWaves < NW, "scale loads need a spare wave");

  // One LDS variable per stage: the compiler then knows that reading stage g
  // does not touch the buffers whose direct-to-LDS loads are still in flight,
  // and does not wait for those loads before the reads (with one array
  // indexed by g % STAGES it must assume they alias and drain every load).
  __shared__ __attribute__((aligned(1024))) uint8_t smem0[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t smem1[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t smem2[STAGES > 2 ? kStage : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t smem3[STAGES > 3 ? kStage : 16];
  auto stage_buf = [&](int s) -> uint8_t* {
    return s == 0 ? smem0 : s == 1 ? smem1 : s == 2 ? smem2 : smem3;
  };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave % WN, wm = wave / WN;
  const int M = a.m, N = a.n, K = a.k;
  const int KG = K >> 7;
  const int NB = (N + 127) >> 7;
  const int tiles_n = (N + BN - 1) / BN, tiles_m = (M + BM - 1) / BM;
  // logical (tile, split) of this workgroup: consecutive tiles of one split
  // share an XCD, so the tiles reading the same A rows or B rows meet in its L2
  const int L = xcd_contiguous((int)(blockIdx.y * gridDim.x + blockIdx.x), (int)(gridDim.x * gridDim.y));
  const int tile = L % (int)gridDim.x;
  int tn, tm;
  // mend: end of the tile's rows; bq/bs: the weights (the expert's, grouped)
  int n0, m0, mend;
  const uint8_t* bq = a.bq;
  const float* bs = a.bs;
  if constexpr (GROUPED) {
    int e, r0, r1;
    if (!grouped_tile<BM>(a, tile / tiles_n, lane, &e, &r0, &r1)) return;
    tn = tile % tiles_n;
    n0 = tn * BN;
    m0 = r0;
    mend = r1;
    bq += (int64_t)e * N * K;
    bs += (int64_t)e * NB * KG;
  } else {
    tile_of(tile, tiles_n, tiles_m, &tn, &tm);
    n0 = tn * BN;
    m0 = tm * BM;
    mend = M;
  }
  // split-K: split z covers a contiguous range of scale groups
  const int split = gridDim.y, z = L / (int)gridDim.x;
  const int gb = (int)((int64_t)z * KG / split), ge = (int)((int64_t)(z + 1) * KG / split);
  const int NG = ge - gb;
  // tile buffers: rows past the last row of A or B read as zeros
  const int nrows = min(BN, N - n0), mrows = min(BM, mend - m0);
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(bq + (int64_t)n0 * K, (uint32_t)(nrows * K));
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(a.aq + (int64_t)m0 * K, (uint32_t)(mrows * K));
  const int mlast = mend - 1 - m0;  // last valid row inside the tile

  // direct-to-LDS slots: wave instruction r covers rows 8*(wave + r*NW) .. +8;
  // lane -> row + (lane >> 3), chunk (lane & 7) ^ (lane >> 3).  The per-lane
  // offset is the same for every instruction; the row block and the scale
  // group go into the scalar offset.
  const int lrow = lane >> 3;
  const int loff = lrow * K + ((lane & 7) ^ lrow) * 16;
  const int rsub = lane & 15, c0 = lane >> 4;
  // scale loads: waves 0 .. kSaWaves-1 fetch 64 activation scales each (one
  // per lane, row wave*64 + lane), the other waves fetch the weight scale of the
  // tile's first 128-row block (every wave of the tile shares it when BN <=
  // 128; otherwise each wave reads its own block's scale, see below)
  const bool sa_wave = wave < kSaWaves;
  const float* scale_src;
  int scale_dst;
  if (sa_wave) {
    scale_src = a.as + (int64_t)(m0 + min(wave * 64 + lane, mlast)) * KG;
    scale_dst = kOffSA + wave * 256;
  } else {
    // lanes 0..kSbBlocks-1 fetch the weight scales of the tile's blocks
    constexpr int kSbBlocks = BN >= 128 ? BN / 128 : 1;  // weight blocks the tile spans
    const int nb = min((n0 >> 7) + min(lane, kSbBlocks - 1), NB - 1);
    scale_src = bs + (int64_t)nb * KG;
    scale_dst = kOffSB;
  }

  auto issue_stage = [&](int g, uint8_t* sb) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(scale_src + g),
                                     (__attribute__((address_space(3))) void*)(sb + scale_dst), 4,
                                     0, 0);
#pragma unroll
    for (int r = 0; r < RB; ++r)
      buffer_to_lds16(rB, sb + 8 * (wave + r * NW) * 128, loff, 8 * (wave + r * NW) * K + g * 128);
#pragma unroll
    for (int r = 0; r < RA; ++r) {
      const int blk = (wave + r * NW) % kABlocks;
      buffer_to_lds16(rA, sb + kOffA + 8 * blk * 128, loff, 8 * blk * K + g * 128);
    }
  };

  f32x4 acc[SN][SM];
#pragma unroll
  for (int i = 0; i < SN; ++i)
#pragma unroll
    for (int j = 0; j < SM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // local group g (scale group gb + g) lives in stage buffer g % STAGES
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < NG) issue_stage(gb + d, stage_buf(d));

  // the loop is unrolled by STAGES so every buffer index is a constant
  for (int g0 = 0; g0 < NG; g0 += STAGES) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s) {
    const int g = g0 + s;
    if (g >= NG) break;
    // stage g must have landed; the D-1 later stages may still be in flight.
    // After the barrier every wave's share of stage g is in LDS and stage g-1
    // (whose buffer the next issue overwrites) has been read by all waves.
    if (g + D - 1 < NG) {
      stage_barrier<(D - 1) * kLoadsPerStage>();
    } else {
      stage_barrier<0>();
    }
    if (g + D < NG) issue_stage(gb + g + D, stage_buf((s + D) % STAGES));

    const uint8_t* st = stage_buf(s);
    const uint8_t* bB = st;
    const uint8_t* bA = st + kOffA;
    const float* sA = reinterpret_cast<const float*>(st + kOffSA);
    const float sbC = reinterpret_cast<const float*>(st + kOffSB)[(wn * TN) >> 7];
    i32x8 aop[SM];
#pragma unroll
    for (int j = 0; j < SM; ++j) aop[j] = lds_operand(bA, wm * TM + 16 * j + rsub, c0);
    float sab[SM];
#pragma unroll
    for (int j = 0; j < SM; ++j) sab[j] = sA[wm * TM + 16 * j + rsub] * sbC;
    // the MFMAs of weight slice i are independent of the promotion FMAs of
    // slice i-1, so the matrix core and the VALU overlap (the scheduler
    // interleaves them; the second wave on the SIMD fills the rest).  All SM
    // MFMAs of a slice are issued before their promotions, so a promotion
    // reads a partial three MFMAs after it was issued instead of right
    // behind it (no wait states; 1.5-3% on the 256x256 tiles, one more
    // spilled register outside the group loop)
    constexpr int PJ = SM;
#pragma unroll
    for (int i = 0; i < SN; ++i) {
      const i32x8 bop = lds_operand(bB, wn * TN + 16 * i + rsub, c0);
#pragma unroll
      for (int j0 = 0; j0 < SM; j0 += PJ) {
        f32x4 pv[PJ];
#pragma unroll
        for (int j = 0; j < PJ; ++j) pv[j] = mfma_group(bop, aop[j0 + j]);
#pragma unroll
        for (int j = 0; j < PJ; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[i][j0 + j][r] = __builtin_fmaf(pv[j][r], sab[j0 + j], acc[i][j0 + j][r]);
      }
    }
    }
  }

  if (split > 1) {
    f32x4 part[SN * SM];
#pragma unroll
    for (int i = 0; i < SN; ++i)
#pragma unroll
      for (int j = 0; j < SM; ++j) part[i * SM + j] = acc[i][j];
    auto valid = [&](int q) { return m0 + wm * TM + 16 * (q % SM) + rsub < mend; };
    if (!splitk_fixup<SN * SM>(a, part, split, z, tile, (int64_t)gridDim.x,
                               NW * SN * SM, wave * SN * SM, lane, valid))
      return;
#pragma unroll
    for (int i = 0; i < SN; ++i)
#pragma unroll
      for (int j = 0; j < SM; ++j) acc[i][j] = part[i * SM + j];
  }

  if constexpr (OUT_DT == kFp32) {
#pragma unroll
    for (int i = 0; i < SN; ++i)
#pragma unroll
      for (int j = 0; j < SM; ++j) {
        const int m = m0 + wm * TM + 16 * j + rsub;
        if (m < mend) store_out4<OUT_DT>(a, m, n0 + wn * TN + 16 * i + 4 * c0, acc[i][j]);
      }
  } else {
    // 16-bit outputs leave through LDS: each lane's four consecutive outputs
    // go to the C tile in LDS (rows padded by 8 bytes so the 16 rows of a
    // store phase fall in different banks), then every row of the tile is
    // written to C as contiguous 16-byte pieces.
    using OT = typename OutT<OUT_DT>::T;
    constexpr int kRow = BN * 2 + 8;
    constexpr int kRowsPerBuf = kStage / kRow;  // C-tile rows in one stage buffer
    static_assert(STAGES * kRowsPerBuf >= BM, "C tile must fit in the stage buffers");
    auto crow = [&](int ml) -> uint8_t* {
      const int b = ml / kRowsPerBuf;
      return stage_buf(b) + (ml - b * kRowsPerBuf) * kRow;
    };
    stage_barrier<0>();  // all waves are done with the stage buffers
#pragma unroll
    for (int i = 0; i < SN; ++i)
#pragma unroll
      for (int j = 0; j < SM; ++j) {
        const int ml = wm * TM + 16 * j + rsub, nl = wn * TN + 16 * i + 4 * c0;
        typedef OT ot4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<ot4*>(crow(ml) + nl * 2) =
            ot4{to_out<OUT_DT>(acc[i][j][0]), to_out<OUT_DT>(acc[i][j][1]),
                to_out<OUT_DT>(acc[i][j][2]), to_out<OUT_DT>(acc[i][j][3])};
      }
    stage_barrier<0>();
    constexpr int kChunks = BN / 8;  // 16-byte pieces per tile row
    OT* C = reinterpret_cast<OT*>(a.c);
    const bool vec = a.vec_ok && (N % 8) == 0;
    for (int idx = threadIdx.x; idx < BM * kChunks; idx += 64 * NW) {
      const int ml = idx / kChunks, cc = idx % kChunks;
      const int m = m0 + ml, n = n0 + cc * 8;
      if (m >= mend || n >= N) continue;
      const uint8_t* src = crow(ml) + cc * 16;
      OT* dst = C + (int64_t)m * N + n;
      if (vec && n + 7 < N) {
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(src),
                                    reinterpret_cast<u32x4*>(dst));
      } else {
        const OT* e = reinterpret_cast<const OT*>(src);
        for (int r = 0; r < 8 && n + r < N; ++r) dst[r] = e[r];
      }
    }
  }
}

// ---- persistent prefill kernel with load and store roles ---------------------------
// grid: P workgroups (one per CU, two for 128x128 tiles).  Workgroup b walks
// the output tiles u = lb, lb + P, lb + 2P, ... with lb its XCD-contiguous
// number, so in every round the P tiles in flight are consecutive and each XCD
// owns a contiguous, M-grouped block of them.  Requires an even number of
// scale groups, so group g of any tile lives in stage buffer g % 2.
//
// The first half of the waves issue every direct-to-LDS stage load and the
// second half every global store of the output.  A wave's vector memory
// counter counts loads and stores in issue order, so a wave that waits for its
// stage loads would also wait for any store it issued earlier; with the roles
// split, the loading waves never have stores outstanding and the storing
// waves never wait on the counter, and a tile's stores drain while the next
// tiles are multiplied.  All waves multiply.  Across tiles the pipeline does
// not stop: the next tile's first group streams in while the last group of
// the current one is multiplied, and the output tile is staged through the
// just-consumed stage buffer in passes of RP rows, which the storing waves
// read into registers and store without waiting for the stores.
//
// The loads are inline assembly (asm_buffer_to_lds16) and the loading
// waves spread a stage's loads over the weight slices of the group being
// multiplied, so issuing them does not hold back that wave's MFMAs.

// Largest bm / 2^i that fits in `fit` rows (the C tile leaves in equal passes).
__host__ __device__ constexpr int pass_rows(int bm, int fit) {
  return (bm <= fit || bm <= 16) ? bm : pass_rows(bm / 2, fit);
}

template <int BN, int BM, int WN, int WM, int OUT_DT, bool GROUPED = false>
__global__ __launch_bounds__(64 * WN * WM) void gemm_persist_kernel(GemmArgs a) {
  using OT = typename OutT<OUT_DT>::T;
  constexpr int NW = WN * WM;
  constexpr int NL = NW / 2;  // loading waves 0 .. NL-1, storing waves NL .. NW-1
  constexpr int NS = NW - NL;
  constexpr int TN = BN / WN, TM = BM / WM;
  constexpr int SN = TN / 16, SM = TM / 16;
  constexpr int kOffA = BN * 128;
  constexpr int kOffSA = (BN + BM) * 128;
  constexpr int kSaBlocks = (BM + 63) / 64;  // 64-row blocks of activation scales
  constexpr int kOffSB = kOffSA + kSaBlocks * 256;
  constexpr int kStage = ((kOffSB + 256) + 1023) / 1024 * 1024;
  constexpr int RB = BN / 8 / NL;  // weight row blocks per loading wave per stage
  constexpr int RA = BM / 8 / NL;  // activation row blocks per loading wave per stage
  constexpr int kLoads = 2 + RB + RA;  // per loading wave per stage
  constexpr int kPerSlice = (kLoads + SN - 2) / (SN - 1);
  constexpr int kOB = (int)sizeof(OT);
  constexpr int kRow = BN * kOB + (kOB == 2 ? 8 : 16);  // padded C row in LDS
  constexpr int RP = pass_rows(BM, kStage / kRow);       // C rows per pass
  constexpr int kChunks = BN * kOB / 16;                 // 16-byte pieces per C row
  constexpr int kPieces = RP * kChunks / (64 * NS);      // per storing lane per pass
  static_assert(NW % 2 == 0, "even wave count");
  static_assert(TN % 16 == 0 && TM % 16 == 0 && SN >= 2, "wave tile of 16-row slices");
  static_assert(128 % TN == 0, "a wave must stay inside one 128-row weight block");
  static_assert(BN >= 128 ? BN % 128 == 0 : 128 % BN == 0, "tiles align to weight blocks");
  static_assert(BN % (8 * NL) == 0 && BM % (8 * NL) == 0, "row blocks split over the loaders");
  static_assert(BM % 64 == 0 && kSaBlocks <= NL, "one activation-scale block per loader");
  static_assert(RP % 16 == 0 && BM % RP == 0, "C passes cover whole 16-row slices");
  static_assert((RP * kChunks) % (64 * NS) == 0, "C pass splits over the storers");

  __shared__ __attribute__((aligned(1024))) uint8_t smem0[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t smem1[kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Grouped tiles with two waves per SIMD: wave rows from the bottom of the
  // tile up, so that in an expert's last tile, which often ends early, the
  // waves with no rows left are the loading ones (0 .. NL-1); they skip the
  // multiply and only issue loads, and the busy wave on each SIMD has the
  // matrix core to itself (32 experts, N=4096, K=7168, 4096 rows on 256x256
  // tiles: 270.7 -> 250 us; 2048 rows 242 -> 220 us).  With one wave per
  // SIMD (128x128 tiles) nothing is gained and it measured 4% slower; the
  // plain GEMM keeps top-down rows (the reversed order spills 64 more
  // registers there).
  constexpr bool kSkipIdle = GROUPED && NW >= 8;
  const int wn = wave % WN, wm = kSkipIdle ? WM - 1 - wave / WN : wave / WN;
  const int M = a.m, N = a.n, K = a.k;
  const int KG = K >> 7;
  const int NB = (N + 127) >> 7;
  const int tiles_n = (N + BN - 1) / BN, tiles_m = (M + BM - 1) / BM;
  // grouped: the experts' M tiles, each with every N tile (N tile fastest)
  const int tiles = tiles_n * (GROUPED ? grouped_mtiles<BM>(a, lane) : tiles_m);
  const int P = gridDim.x;
  // Work units: whole tiles, except that with a tail split S > 1 (plain GEMM)
  // the `tail` tiles of the last, partial round (all tiles when there are
  // fewer than P) are each cut into S K ranges of whole pairs of scale groups,
  // one unit each (the host keeps tail * S <= P, so they run in one round).
  const int S = (!GROUPED && a.tail_split > 1) ? a.tail_split : 1;
  const int full = S > 1 ? tiles / P * P : tiles;
  const int tail = tiles - full;
  const int units = full + tail * S;
  int u = xcd_contiguous((int)blockIdx.x, P);
  if (u >= units) return;
  // tile uu: first column n0, rows [m0, mend), expert e (0 when not grouped)
  auto tile_at = [&](int uu, int* n0, int* m0, int* mend, int* e) {
    if constexpr (GROUPED) {
      (void)grouped_tile<BM>(a, uu / tiles_n, lane, e, m0, mend);
      *n0 = (uu % tiles_n) * BN;
    } else {
      int tn, tm;
      tile_of(uu, tiles_n, tiles_m, &tn, &tm);
      *n0 = tn * BN;
      *m0 = tm * BM;
      *mend = M;
      *e = 0;
    }
  };

  // unit uu: its tile (tile_at), the scale groups [gb, ge) it adds up and,
  // for a piece of a cut tile, the piece z and the tile's tail index tt
  // (tt = -1 for a whole tile).  Consecutive pieces are different tiles at the
  // same K range, so an XCD's pieces share A or B rows in its L2.
  const int NP = KG >> 1;
  auto unit_at = [&](int uu, int* n0, int* m0, int* mend, int* e, int* gb, int* ge, int* z,
                     int* tt) {
    int t = uu, zz = 0, s = 1;
    *tt = -1;
    if (uu >= full) {
      const int v = uu - full;
      t = full + v % tail;
      zz = v / tail;
      s = S;
      *tt = v % tail;
    }
    tile_at(t, n0, m0, mend, e);
    *z = zz;
    *gb = 2 * (int)((int64_t)zz * NP / s);
    *ge = 2 * (int)((int64_t)(zz + 1) * NP / s);
  };

  const int lrow = lane >> 3;
  const int loff = lrow * K + ((lane & 7) ^ lrow) * 16;
  const int rsub = lane & 15, c0 = lane >> 4;

  f32x4 acc[SN][SM];
  // one scale group from stage buffer st; between(i) runs after the MFMAs of
  // weight slice i
  auto compute = [&](const uint8_t* st, auto between) {
    const uint8_t* bB = st;
    const uint8_t* bA = st + kOffA;
    const float* sA = reinterpret_cast<const float*>(st + kOffSA);
    // Plain GEMM: the weight operand of slice i+1 is read while slice i is
    // multiplied, so its LDS latency is not waited out before the slice's
    // first MFMA (256x256 tiles: 7168x16384 470 -> 459 us, 24576x1536
    // 167 -> 163 us), and the first slice's operands are read ahead of the
    // scales, so the group's first MFMA does not wait for the scale reads
    // (LDS returns in order; 7168x16384 471 -> 468 us).  The grouped forms
    // keep the read in the slice: with the prefetch they lost time (32
    // experts, N=4096, K=7168: 2 rows per expert on 128x128 tiles 152 -> 177
    // us, 128 rows on 256x256 254 -> 261 us).
    constexpr bool kPrefetch = !GROUPED;
    i32x8 bnext{};
    if constexpr (kPrefetch) bnext = lds_operand(bB, wn * TN + rsub, c0);
    i32x8 aop[SM];
#pragma unroll
    for (int j = 0; j < SM; ++j) aop[j] = lds_operand(bA, wm * TM + 16 * j + rsub, c0);
    const float sbC = reinterpret_cast<const float*>(st + kOffSB)[(wn * TN) >> 7];
    float sab[SM];
#pragma unroll
    for (int j = 0; j < SM; ++j) sab[j] = sA[wm * TM + 16 * j + rsub] * sbC;
    // Plain GEMM: all SM MFMAs of a slice before their promotion FMAs, so
    // each partial is read several MFMAs after it was issued, with no wait
    // states (24576x1536 188.7 -> 184.7 us, 7168x16384 472.7 -> 465.7,
    // 4096^3 74.9 -> 72.7; same box, alternating builds).  The grouped forms,
    // which hold more state, keep pairs: four spilled 16-32 more bytes there.
    constexpr int PJ = (GROUPED && SM >= 4) ? 2 : SM;
#pragma unroll
    for (int i = 0; i < SN; ++i) {
      i32x8 bop;
      if constexpr (kPrefetch) {
        bop = bnext;
        if (i + 1 < SN) bnext = lds_operand(bB, wn * TN + 16 * (i + 1) + rsub, c0);
      } else {
        bop = lds_operand(bB, wn * TN + 16 * i + rsub, c0);
      }
#pragma unroll
      for (int j0 = 0; j0 < SM; j0 += PJ) {
        f32x4 pv[PJ];
#pragma unroll
        for (int j = 0; j < PJ; ++j) pv[j] = mfma_group(bop, aop[j0 + j]);
#pragma unroll
        for (int j = 0; j < PJ; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[i][j0 + j][r] = __builtin_fmaf(pv[j][r], sab[j0 + j], acc[i][j0 + j][r]);
      }
      between(i);
    }
  };
  // Keep a group's MFMAs ahead of the next barrier: otherwise the compiler
  // may sink them next to the following group's operand reads and spill.
  auto pin_acc = [&]() {
#pragma unroll
    for (int i = 0; i < SN; ++i)
#pragma unroll
      for (int j = 0; j < SM; ++j) asm volatile("" : "+v"(acc[i][j]));
  };

  // The roles run separate copies of the loop, so the compiler's own wait
  // analysis never sees a load on a storing wave's path or a store on a
  // loading wave's path.
  auto run = [&](auto role) {
    constexpr bool kLoader = decltype(role)::value;
    // loading waves wait for their loads; storing waves have none
    auto barrier = [&]() {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(kLoader ? 0 : 63));
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    // the output passes only synchronize LDS: no wait for vector memory (the
    // next unit's first group has landed at the barrier before them, and the
    // stores of C need not complete)
    auto lds_barrier = [&]() {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(63));
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    const int l = kLoader ? wave : 0;
    u32x4 rB = u32x4{0u, 0u, 0u, 0u}, rA = u32x4{0u, 0u, 0u, 0u};
    const float* sa_src = a.as;
    const float* sb_src = a.bs;
    // tile buffers: rows past the last row of A or B read as zeros
    auto set_loads = [&](int n0, int m0, int mend, int e) {
      if constexpr (kLoader) {
        const int nrows = min(BN, N - n0), mrows = min(BM, mend - m0);
        rB = rsrc_words(a.bq + ((int64_t)e * N + n0) * K, (uint32_t)(nrows * K));
        rA = rsrc_words(a.aq + (int64_t)m0 * K, (uint32_t)(mrows * K));
        sa_src = a.as + (int64_t)(m0 + min(min(l, kSaBlocks - 1) * 64 + lane, mend - 1 - m0)) * KG;
        constexpr int kSbBlocks = BN >= 128 ? BN / 128 : 1;
        const int nb = min((n0 >> 7) + min(lane, kSbBlocks - 1), NB - 1);
        sb_src = a.bs + ((int64_t)e * NB + nb) * KG;
      }
    };
    // Load d of a stage: 0 the activation scales, 1 the weight scales, then
    // RB weight and RA activation row blocks.  Every loader issues the same
    // loads (loaders past the last activation-scale block repeat it, and all
    // write the same weight scales), which the stage barrier's count assumes.
    auto issue_load = [&](int g, uint8_t* sb, int d) {
      if constexpr (kLoader) {
        const uint32_t base = lds_addr(sb);
        if (d == 0) {
          asm_global_to_lds4(sa_src + g, base + kOffSA + min(l, kSaBlocks - 1) * 256);
        } else if (d == 1) {
          asm_global_to_lds4(sb_src + g, base + kOffSB);
        } else if (d < 2 + RB) {
          const int r = d - 2;
          asm_buffer_to_lds16(rB, base + 8 * (l + r * NL) * 128, loff,
                              8 * (l + r * NL) * K + g * 128);
        } else {
          const int r = d - 2 - RB;
          asm_buffer_to_lds16(rA, base + kOffA + 8 * (l + r * NL) * 128, loff,
                              8 * (l + r * NL) * K + g * 128);
        }
      }
    };
    // stage g's loads, kPerSlice after each of the first weight slices
    auto spread = [&](int g, uint8_t* sb) {
      return [&, g, sb](int i) {
#pragma unroll
        for (int q = 0; q < kPerSlice; ++q)
          if (i * kPerSlice + q < kLoads) issue_load(g, sb, i * kPerSlice + q);
      };
    };

    int n0, m0, mend, ex, gb, ge, z, tt;
    unit_at(u, &n0, &m0, &mend, &ex, &gb, &ge, &z, &tt);
    set_loads(n0, m0, mend, ex);
#pragma unroll
    for (int d = 0; d < kLoads; ++d) issue_load(gb, smem0, d);
    barrier();
    for (;;) {
      const int nu = u + P;
      const bool has_next = nu < units;
      int nn0 = n0, nm0 = m0, nmend = mend, nex = ex, ngb = gb, nge = ge, nz = z, ntt = tt;
      if (has_next) unit_at(nu, &nn0, &nm0, &nmend, &nex, &ngb, &nge, &nz, &ntt);
#pragma unroll
      for (int i = 0; i < SN; ++i)
#pragma unroll
        for (int j = 0; j < SM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      // (kSkipIdle) a wave whose rows all lie past the tile's last row
      // multiplies nothing: its accumulators stay zero and its rows are never
      // stored; it still issues its share of the loads.
      const bool busy = !kSkipIdle || m0 + wm * TM < mend;
      auto step = [&](const uint8_t* st, auto between) {
        if (busy) {
          compute(st, between);
        } else {
#pragma unroll
          for (int i = 0; i < SN; ++i) between(i);
        }
      };
      // on entry group gb of the unit is in buffer 0 (gb and ge are even)
      for (int g0 = gb; g0 + 2 < ge; g0 += 2) {
        step(smem0, spread(g0 + 1, smem1));
        pin_acc();
        barrier();  // group g0 + 1 landed; every wave is done with buffer 0
        step(smem1, spread(g0 + 2, smem0));
        pin_acc();
        barrier();  // group g0 + 2 landed; every wave is done with buffer 1
      }
      step(smem0, spread(ge - 1, smem1));
      pin_acc();
      barrier();  // group ge - 1 landed; every wave is done with buffer 0
      // the next unit's first group (the last unit reloads its own, which
      // keeps the group free of branches)
      set_loads(nn0, nm0, nmend, nex);
      step(smem1, spread(ngb, smem0));
      pin_acc();
      barrier();  // the next unit's first group landed; buffer 1 is free

      if (tt >= 0) {
        // a piece of a cut tile (always a workgroup's last unit): its fp32
        // partial goes to the workspace in this wave's register layout, one
        // 1 KB store per pair; the tail kernel adds the pieces.  Plain
        // stores: the tail kernel reads the partials right after this launch,
        // and with the non-temporal hint it took 2-4 us longer (M=4096,
        // N=4608, K=7168: 138 -> 134 us; M=1024, N=36864: 271 -> 267 us).
        const int64_t base = ((((int64_t)z * tail + tt) * NW + wave) * (SN * SM)) * 64 + lane;
        f32x4* part = reinterpret_cast<f32x4*>(a.ws) + base;
#pragma unroll
        for (int i = 0; i < SN; ++i)
#pragma unroll
          for (int j = 0; j < SM; ++j) part[(i * SM + j) * 64] = acc[i][j];
        break;
      }

      // the output tile leaves through buffer 1, RP rows per pass
      OT* C = reinterpret_cast<OT*>(a.c);
      const bool vec = a.vec_ok && (N % (16 / kOB)) == 0;
#pragma unroll
      for (int p = 0; p < BM / RP; ++p) {
#pragma unroll
        for (int j = 0; j < SM; ++j) {
          const int sr = wm * TM + 16 * j;  // first tile row of the slice
          if (sr < p * RP || sr >= (p + 1) * RP) continue;
#pragma unroll
          for (int i = 0; i < SN; ++i) {
            const int nl = wn * TN + 16 * i + 4 * c0;
            uint8_t* dst = smem1 + (sr - p * RP + rsub) * kRow + nl * kOB;
            if constexpr (kOB == 4) {
              *reinterpret_cast<f32x4*>(dst) = acc[i][j];
            } else {
              typedef OT ot4 __attribute__((ext_vector_type(4)));
              *reinterpret_cast<ot4*>(dst) =
                  ot4{to_out<OUT_DT>(acc[i][j][0]), to_out<OUT_DT>(acc[i][j][1]),
                      to_out<OUT_DT>(acc[i][j][2]), to_out<OUT_DT>(acc[i][j][3])};
            }
          }
        }
        lds_barrier();  // the pass is in LDS
        if constexpr (!kLoader) {
          // four pieces at a time: the accumulators of later passes are live
          constexpr int QB = kPieces < 4 ? kPieces : 4;
          static_assert(kPieces % QB == 0, "C pieces in batches");
#pragma unroll
          for (int q0 = 0; q0 < kPieces; q0 += QB) {
            u32x4 piece[QB];
#pragma unroll
            for (int q = 0; q < QB; ++q) {
              const int idx = (wave - NL) * 64 + lane + (q0 + q) * 64 * NS;
              piece[q] = *reinterpret_cast<const u32x4*>(smem1 + (idx / kChunks) * kRow +
                                                         (idx % kChunks) * 16);
            }
#pragma unroll
            for (int q = 0; q < QB; ++q) {
              const int idx = (wave - NL) * 64 + lane + (q0 + q) * 64 * NS;
              const int m = m0 + p * RP + idx / kChunks, n = n0 + (idx % kChunks) * (16 / kOB);
              if (m >= mend || n >= N) continue;
              OT* dst = C + (int64_t)m * N + n;
              if (vec && n + 16 / kOB - 1 < N) {
                __builtin_nontemporal_store(piece[q], reinterpret_cast<u32x4*>(dst));
              } else {
                const OT* e = reinterpret_cast<const OT*>(&piece[q]);
                for (int r = 0; r < 16 / kOB && n + r < N; ++r) dst[r] = e[r];
              }
            }
          }
        }
        lds_barrier();  // the storing waves have read the pass out of LDS
      }
      if (!has_next) break;
      u = nu;
      n0 = nn0;
      m0 = nm0;
      mend = nmend;
      ex = nex;
      gb = ngb;
      ge = nge;
      z = nz;
      tt = ntt;
    }
  };
  if (wave < NL) {
    run(std::integral_constant<bool, true>{});
  } else {
    run(std::integral_constant<bool, false>{});
  }
}

// ---- tail reduction of the persistent kernel ---------------------------------------
// One thread per (cut tile, wave, pair, lane) slot of the partial layout the
// persistent kernel stores: the S pieces' four fp32 values are added in piece
// order (deterministic) and the four outputs stored.  The slot's output
// position follows the persistent kernel's wave tiling.
template <int BN, int BM, int WN, int WM, int OUT_DT>
__global__ __launch_bounds__(256) void gemm_tail_reduce_kernel(GemmArgs a, int full, int tail) {
  constexpr int NW = WN * WM;
  constexpr int TN = BN / WN, TM = BM / WM;
  constexpr int SN = TN / 16, SM = TM / 16;
  constexpr int kSlots = NW * SN * SM * 64;  // per tile
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)tail * kSlots) return;
  const int tt = (int)(t / kSlots);
  const int r = (int)(t - (int64_t)tt * kSlots);
  const int lane = r & 63, q = (r >> 6) % (SN * SM), wave = (r >> 6) / (SN * SM);
  const int i = q / SM, j = q % SM, wn = wave % WN, wm = wave / WN;
  const int tiles_n = (a.n + BN - 1) / BN, tiles_m = (a.m + BM - 1) / BM;
  int tn, tm;
  tile_of(full + tt, tiles_n, tiles_m, &tn, &tm);
  const int m = tm * BM + wm * TM + 16 * j + (lane & 15);
  const int n = tn * BN + wn * TN + 16 * i + 4 * (lane >> 4);
  if (m >= a.m) return;
  const f32x4* part = reinterpret_cast<const f32x4*>(a.ws) + (int64_t)tt * kSlots + r;
  const int64_t piece = (int64_t)tail * kSlots;
  f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int z = 0; z < a.tail_split; ++z) sum += __builtin_nontemporal_load(part + z * piece);
  store_out4<OUT_DT>(a, m, n, sum);
}

// ---- kernel table -------------------------------------------------------------

using KernelFn = void (*)(GemmArgs);

struct CfgEntry {
  int kind;  // 1 = decode, 2 = prefill, 3 = persistent prefill, 4 = wide decode
  int bn, bm, waves;
  const char* name;
  KernelFn fn[3];  // [out_dt index]
  // tiled (kind 2) and persistent (kind 3): the grouped-expert variant, where
  // built (else null); wide decode (kind 4): the variant without the scale
  // preload, for more than wide_scale_cap() groups per wave
  KernelFn fn_alt[3];
  // wide decode (kind 4): the grouped-expert variants with and without the
  // scale preload, where built (else null)
  KernelFn fn_grp[3];
  KernelFn fn_grp_alt[3];
  // persistent (kind 3): the reduction of cut tail tiles
  void (*fn_tail[3])(GemmArgs, int, int);
};

#define DECODE_CFG(MT, WK, U, NAME)                                                           \
  {1, 16, 16 * MT, WK, NAME,                                                                   \
   {gemm_decode_kernel<MT, WK, U, kFp32>, gemm_decode_kernel<MT, WK, U, kFp16>,                \
    gemm_decode_kernel<MT, WK, U, kBf16>}}
#define DECODE_LDS_CFG(WK, U, NAME)                                                            \
  {1, 16, 16, WK, NAME,                                                                        \
   {gemm_decode_lds_kernel<WK, U, kFp32>, gemm_decode_lds_kernel<WK, U, kFp16>,                \
    gemm_decode_lds_kernel<WK, U, kBf16>}}
#define PREFILL_CFG(BN, BM, WN, WM, ST, NAME)                                                 \
  {2, BN, BM, WN * WM, NAME,                                                                   \
   {gemm_prefill_kernel<BN, BM, WN, WM, ST, kFp32>,                                            \
    gemm_prefill_kernel<BN, BM, WN, WM, ST, kFp16>,                                            \
    gemm_prefill_kernel<BN, BM, WN, WM, ST, kBf16>}}

#define PREFILL_GROUPED_CFG(BN, BM, WN, WM, ST, NAME)                                         \
  {2,                                                                                          \
   BN,                                                                                         \
   BM,                                                                                         \
   WN * WM,                                                                                    \
   NAME,                                                                                       \
   {gemm_prefill_kernel<BN, BM, WN, WM, ST, kFp32>,                                            \
    gemm_prefill_kernel<BN, BM, WN, WM, ST, kFp16>,                                            \
    gemm_prefill_kernel<BN, BM, WN, WM, ST, kBf16>},                                           \
   {gemm_prefill_kernel<BN, BM, WN, WM, ST, kFp32, true>,                                      \
    gemm_prefill_kernel<BN, BM, WN, WM, ST, kFp16, true>,                                      \
    gemm_prefill_kernel<BN, BM, WN, WM, ST, kBf16, true>}}
#define DECODE_WIDE_CFG(MT, WK, UW, UA, NAME)                                                  \
  {4,                                                                                          \
   16,                                                                                         \
   16 * MT,                                                                                    \
   WK,                                                                                         \
   NAME,                                                                                       \
   {gemm_decode_wide_kernel<MT, WK, UW, UA, true, kFp32>,                                      \
    gemm_decode_wide_kernel<MT, WK, UW, UA, true, kFp16>,                                      \
    gemm_decode_wide_kernel<MT, WK, UW, UA, true, kBf16>},                                     \
   {gemm_decode_wide_kernel<MT, WK, UW, UA, false, kFp32>,                                     \
    gemm_decode_wide_kernel<MT, WK, UW, UA, false, kFp16>,                                     \
    gemm_decode_wide_kernel<MT, WK, UW, UA, false, kBf16>}}
#define DECODE_WIDE_GCFG(MT, WK, UW, UA, NAME)                                                 \
  {4,                                                                                          \
   16,                                                                                         \
   16 * MT,                                                                                    \
   WK,                                                                                         \
   NAME,                                                                                       \
   {gemm_decode_wide_kernel<MT, WK, UW, UA, true, kFp32>,                                      \
    gemm_decode_wide_kernel<MT, WK, UW, UA, true, kFp16>,                                      \
    gemm_decode_wide_kernel<MT, WK, UW, UA, true, kBf16>},                                     \
   {gemm_decode_wide_kernel<MT, WK, UW, UA, false, kFp32>,                                     \
    gemm_decode_wide_kernel<MT, WK, UW, UA, false, kFp16>,                                     \
    gemm_decode_wide_kernel<MT, WK, UW, UA, false, kBf16>},                                    \
   {gemm_decode_wide_kernel<MT, WK, UW, UA, true, kFp32, true>,                                \
    gemm_decode_wide_kernel<MT, WK, UW, UA, true, kFp16, true>,                                \
    gemm_decode_wide_kernel<MT, WK, UW, UA, true, kBf16, true>},                               \
   {gemm_decode_wide_kernel<MT, WK, UW, UA, false, kFp32, true>,                               \
    gemm_decode_wide_kernel<MT, WK, UW, UA, false, kFp16, true>,                               \
    gemm_decode_wide_kernel<MT, WK, UW, UA, false, kBf16, true>}}
#define DECODE_WIDE_M8CFG(WK, UW, UA, NAME)                                                    \
  {4,                                                                                          \
   16,                                                                                         \
   8,                                                                                          \
   WK,                                                                                         \
   NAME,                                                                                       \
   {gemm_decode_wide_kernel<1, WK, UW, UA, true, kFp32, false, 1, 8>,                          \
    gemm_decode_wide_kernel<1, WK, UW, UA, true, kFp16, false, 1, 8>,                          \
    gemm_decode_wide_kernel<1, WK, UW, UA, true, kBf16, false, 1, 8>},                         \
   {gemm_decode_wide_kernel<1, WK, UW, UA, false, kFp32, false, 1, 8>,                         \
    gemm_decode_wide_kernel<1, WK, UW, UA, false, kFp16, false, 1, 8>,                         \
    gemm_decode_wide_kernel<1, WK, UW, UA, false, kBf16, false, 1, 8>}}
#define DECODE_WIDE_NCFG(NT, MT, WK, UW, UA, NAME)                                             \
  {4,                                                                                          \
   16 * NT,                                                                                    \
   16 * MT,                                                                                    \
   WK,                                                                                         \
   NAME,                                                                                       \
   {gemm_decode_wide_kernel<MT, WK, UW, UA, true, kFp32, false, NT>,                           \
    gemm_decode_wide_kernel<MT, WK, UW, UA, true, kFp16, false, NT>,                           \
    gemm_decode_wide_kernel<MT, WK, UW, UA, true, kBf16, false, NT>},                          \
   {gemm_decode_wide_kernel<MT, WK, UW, UA, false, kFp32, false, NT>,                          \
    gemm_decode_wide_kernel<MT, WK, UW, UA, false, kFp16, false, NT>,                          \
    gemm_decode_wide_kernel<MT, WK, UW, UA, false, kBf16, false, NT>}}
#define PERSIST_CFG(BN, BM, WN, WM, NAME)                                                      \
  {3,                                                                                          \
   BN,                                                                                         \
   BM,                                                                                         \
   WN * WM,                                                                                    \
   NAME,                                                                                       \
   {gemm_persist_kernel<BN, BM, WN, WM, kFp32>, gemm_persist_kernel<BN, BM, WN, WM, kFp16>,     \
    gemm_persist_kernel<BN, BM, WN, WM, kBf16>},                                               \
   {gemm_persist_kernel<BN, BM, WN, WM, kFp32, true>,                                          \
    gemm_persist_kernel<BN, BM, WN, WM, kFp16, true>,                                          \
    gemm_persist_kernel<BN, BM, WN, WM, kBf16, true>},                                         \
   {nullptr, nullptr, nullptr},                                                                \
   {nullptr, nullptr, nullptr},                                                                \
   {gemm_tail_reduce_kernel<BN, BM, WN, WM, kFp32>,                                            \
    gemm_tail_reduce_kernel<BN, BM, WN, WM, kFp16>,                                            \
    gemm_tail_reduce_kernel<BN, BM, WN, WM, kBf16>}}

const CfgEntry kCfgs[] = {
    DECODE_CFG(1, 1, 8, "dec_m16_k1_u8"),
    DECODE_CFG(1, 2, 8, "dec_m16_k2_u8"),
    DECODE_CFG(1, 4, 8, "dec_m16_k4_u8"),
    DECODE_CFG(1, 8, 8, "dec_m16_k8_u8"),
    DECODE_CFG(2, 4, 4, "dec_m32_k4_u4"),
    DECODE_CFG(4, 4, 2, "dec_m64_k4_u2"),
    PREFILL_CFG(256, 128, 4, 2, 3, "pre_n256_m128_w8_s3"),
    PREFILL_CFG(128, 256, 2, 4, 3, "pre_n128_m256_w8_s3"),
    PREFILL_GROUPED_CFG(128, 128, 2, 2, 2, "pre_n128_m128_w4_s2"),
    PREFILL_CFG(128, 128, 2, 2, 4, "pre_n128_m128_w4_s4"),
    PREFILL_CFG(256, 256, 2, 4, 2, "pre_n256_m256_w8_s2"),
    PREFILL_GROUPED_CFG(128, 64, 8, 1, 4, "pre_n128_m64_w8_s4"),
    PREFILL_GROUPED_CFG(128, 32, 8, 1, 4, "pre_n128_m32_w8_s4"),
    PREFILL_GROUPED_CFG(128, 16, 8, 1, 4, "pre_n128_m16_w8_s4"),
    PREFILL_CFG(64, 64, 4, 1, 4, "pre_n64_m64_w4_s4"),
    PREFILL_GROUPED_CFG(128, 64, 8, 1, 3, "pre_n128_m64_w8_s3"),
    DECODE_LDS_CFG(2, 4, "decl_k2_u4"),
    DECODE_LDS_CFG(4, 4, "decl_k4_u4"),
    DECODE_LDS_CFG(8, 4, "decl_k8_u4"),
    PERSIST_CFG(256, 256, 2, 4, "per_n256_m256_w8"),
    PERSIST_CFG(256, 128, 4, 2, "per_n256_m128_w8"),
    PERSIST_CFG(128, 128, 2, 2, "per_n128_m128_w4"),
    DECODE_WIDE_GCFG(4, 4, 2, 2, "dw_m64_k4_w2a2"),
    DECODE_WIDE_CFG(4, 2, 4, 2, "dw_m64_k2_w4a2"),
    DECODE_WIDE_GCFG(2, 4, 2, 2, "dw_m32_k4_w2a2"),
    DECODE_WIDE_CFG(1, 2, 8, 8, "dw_m16_k2_w8a8"),
    DECODE_WIDE_GCFG(1, 8, 3, 3, "dw_m16_k8_w3a3"),
    DECODE_WIDE_GCFG(1, 4, 3, 3, "dw_m16_k4_w3a3"),
    DECODE_WIDE_CFG(1, 8, 2, 2, "dw_m16_k8_w2a2"),
    DECODE_WIDE_NCFG(4, 4, 4, 2, 2, "dw_n64_m64_k4_w2a2"),
    DECODE_WIDE_NCFG(2, 4, 4, 2, 2, "dw_n32_m64_k4_w2a2"),
    DECODE_WIDE_NCFG(4, 2, 4, 2, 2, "dw_n64_m32_k4_w2a2"),
    DECODE_WIDE_NCFG(2, 1, 8, 3, 3, "dw_n32_m16_k8_w3a3"),
    DECODE_WIDE_NCFG(2, 2, 8, 2, 2, "dw_n32_m32_k8_w2a2"),
    DECODE_WIDE_M8CFG(8, 4, 4, "dw_m8_k8_w4a4"),
    DECODE_WIDE_M8CFG(4, 4, 4, "dw_m8_k4_w4a4"),
};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

// ---- split-K workspace: a fixed pool of slots per device ---------------------
// A slot holds INFEROP_SPLITK_WS_BYTES of fp32 partials and
// INFEROP_SPLITK_WS_COUNTERS arrival counters.  Each device has
// INFEROP_SPLITK_WS_SLOTS of them; a stream takes the next free slot of its
// device at its first split-K call (the slot's memory is allocated then) and
// keeps it until the process ends -- never grown, replaced, freed or handed to
// another stream, so a HIP graph captured on the stream keeps valid pointers,
// two streams never share partials, and no call waits for the host.  Once a
// device's slots are all taken, further streams get no workspace: the
// automatic tile choice then runs unsplit (inferop_hip_splitk_reserve), and
// a forced split is rejected.  So a process holds at most
// INFEROP_SPLITK_WS_SLOTS x (64 MiB + 64 KiB) per device, however many
// streams it creates and destroys (a new stream at a destroyed stream's
// address finds that stream's slot).  The automatic tile choice stays within
// a slot's capacity; a forced split that needs more is rejected before any
// launch.  The counters start at zero and every launch leaves them at zero
// (the workgroup that completes a tile resets its counter).

__global__ void fill_zero_kernel(int* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

hipError_t launch_fill_zero(int* p, int64_t n, hipStream_t st) {
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

struct Workspace {
  float* partials;
  int* counters;
};

struct WorkspacePool {
  Workspace slot[INFEROP_SPLITK_WS_SLOTS];
  hipStream_t owner[INFEROP_SPLITK_WS_SLOTS];
  int used;  // slots handed out, in order; entries are never changed afterwards
};

std::mutex g_ws_mutex;
WorkspacePool g_ws[64];         // per device ordinal
hipStream_t g_zero_stream[64];  // per device, for captured first calls

// The workspace of stream st on the current device: its slot, or the next
// free one (allocated and its counters zeroed here).  hipErrorOutOfMemory
// when every slot belongs to another stream.
hipError_t get_workspace(hipStream_t st, float** ws, int** cnt) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  WorkspacePool& pool = g_ws[dev];
  for (int i = 0; i < pool.used; ++i) {
    if (pool.owner[i] == st) {
      *ws = pool.slot[i].partials;
      *cnt = pool.slot[i].counters;
      return hipSuccess;
    }
  }
  if (pool.used >= INFEROP_SPLITK_WS_SLOTS) return hipErrorOutOfMemory;
  // First split-K call on this stream.  While the stream is being captured,
  // hipMalloc is only allowed in relaxed capture mode, and the counters are
  // zeroed on a library stream that is not captured (waited for here, once);
  // otherwise the zeroing kernel runs on the caller's stream ahead of the GEMM.
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess) return e;
  const bool capturing = cs != hipStreamCaptureStatusNone;
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  if (capturing) {
    e = hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess) return e;
  }
  char* base = nullptr;
  const size_t bytes = (size_t)INFEROP_SPLITK_WS_BYTES + (size_t)INFEROP_SPLITK_WS_COUNTERS * 4;
  e = hipMalloc(&base, bytes);
  int* counters = reinterpret_cast<int*>(base + INFEROP_SPLITK_WS_BYTES);
  if (e == hipSuccess) {
    if (capturing) {
      if (!g_zero_stream[dev]) e = hipStreamCreateWithFlags(&g_zero_stream[dev], hipStreamNonBlocking);
      if (e == hipSuccess) e = launch_fill_zero(counters, INFEROP_SPLITK_WS_COUNTERS, g_zero_stream[dev]);
      if (e == hipSuccess) e = hipStreamSynchronize(g_zero_stream[dev]);
    } else {
      e = launch_fill_zero(counters, INFEROP_SPLITK_WS_COUNTERS, st);
    }
  }
  if (capturing) {
    const hipError_t e2 = hipThreadExchangeStreamCaptureMode(&mode);
    if (e == hipSuccess) e = e2;
  }
  if (e != hipSuccess) {
    // a failed set-up keeps its memory (it may be in use by a launched fill)
    // but takes no slot
    return e;
  }
  pool.slot[pool.used] = Workspace{reinterpret_cast<float*>(base), counters};
  pool.owner[pool.used] = st;
  ++pool.used;
  *ws = reinterpret_cast<float*>(base);
  *cnt = counters;
  return hipSuccess;
}

// ---- scratch of the allocation-free entry point --------------------------------
// inferop_hip_gemm_w8a8_block_noalloc takes its split-K partials and counters
// from this file-scope array (one copy per GPU, held from module load until the
// process ends) instead of the per-stream workspace, so it never allocates.
// Same layout and capacity as a workspace: partials, then the counters.  In
// host code `scratch` is a host-side stand-in; the device address of each
// GPU's copy comes from hipGetSymbolAddress with that device current, kept in
// g_scratch_ptr, and only that address is ever passed to a kernel.
constexpr size_t kScratchBytes =
    (size_t)INFEROP_SPLITK_WS_BYTES + (size_t)INFEROP_SPLITK_WS_COUNTERS * 4;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::once_flag g_scratch_once[64];
hipError_t g_scratch_err[64];
char* g_scratch_ptr[64];

// The current device's scratch address, looked up on the first call on that
// device, which also zeroes the counters ahead of its GEMM (afterwards every
// launch leaves them at zero): on that call's stream, or -- when the first
// call is being captured -- on the library's own stream in relaxed capture
// mode, waited for here, so the zeroing is never a node of the caller's graph
// and eager calls before any replay find the counters at zero too.
hipError_t get_scratch(hipStream_t st, float** ws, int** cnt) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::call_once(g_scratch_once[dev], [&] {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t r = hipStreamIsCapturing(st, &cs);
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const bool capturing = r == hipSuccess && cs != hipStreamCaptureStatusNone;
    if (capturing) r = hipThreadExchangeStreamCaptureMode(&mode);
    void* ptr = nullptr;
    if (r == hipSuccess) r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (r == hipSuccess && ptr == nullptr) r = hipErrorInvalidSymbol;
    if (r == hipSuccess) {
      g_scratch_ptr[dev] = static_cast<char*>(ptr);
      int* counters = reinterpret_cast<int*>(g_scratch_ptr[dev] + INFEROP_SPLITK_WS_BYTES);
      if (capturing) {
        std::lock_guard<std::mutex> lock(g_ws_mutex);  // guards g_zero_stream
        if (!g_zero_stream[dev]) r = hipStreamCreateWithFlags(&g_zero_stream[dev], hipStreamNonBlocking);
        if (r == hipSuccess) r = launch_fill_zero(counters, INFEROP_SPLITK_WS_COUNTERS, g_zero_stream[dev]);
        if (r == hipSuccess) r = hipStreamSynchronize(g_zero_stream[dev]);
      } else {
        r = launch_fill_zero(counters, INFEROP_SPLITK_WS_COUNTERS, st);
      }
    }
    if (capturing) {
      const hipError_t r2 = hipThreadExchangeStreamCaptureMode(&mode);
      if (r == hipSuccess) r = r2;
    }
    g_scratch_err[dev] = r;
  });
  if (g_scratch_err[dev] != hipSuccess) return g_scratch_err[dev];
  *ws = reinterpret_cast<float*>(g_scratch_ptr[dev]);
  *cnt = reinterpret_cast<int*>(g_scratch_ptr[dev] + INFEROP_SPLITK_WS_BYTES);
  return hipSuccess;
}

// Launch plan of a persistent configuration: grid, the tiles of the last,
// partial round that are cut (tail) and into how many K ranges (split), and
// the fp32 partial bytes they need.  The pieces of all cut tiles must run in
// one round (tail * split <= workgroups) and each keeps a pair of groups.
struct PersistPlan {
  int64_t grid, tail, split, ws_bytes;
};
PersistPlan persist_plan(const CfgEntry& cf, int64_t tiles, int64_t kg, int64_t split, int cus) {
  const int64_t slots = (int64_t)cus * (cf.bn * cf.bm <= 128 * 128 ? 2 : 1);
  PersistPlan p{tiles < slots ? tiles : slots, 0, 1, 0};
  int64_t s = split < 1 ? 1 : split;
  if (s > kg / 2) s = kg / 2;
  if (s <= 1) return p;
  const int64_t tail = tiles >= slots ? tiles % slots : tiles;
  if (tail == 0) return p;
  const int64_t fit = slots / tail;
  if (s > fit) s = fit;
  if (s <= 1) return p;
  p.tail = tail;
  p.split = s;
  p.grid = tiles >= slots ? slots : tiles * s;
  p.ws_bytes = s * tail * cf.bn * cf.bm * 4;
  return p;
}

// Workspace a launch of configuration cf with `split` K partitions needs
// (0 without a split), and whether it fits the fixed capacity.
// A tile's partial is laid out in 16x16 output blocks of 1 KB (the fixup's
// pairs): an 8-row activation tile (the M <= 8 wide decode configurations)
// still takes whole 16-row blocks.
int64_t tile_partial_bytes(const CfgEntry& cf) {
  return (int64_t)((cf.bm + 15) / 16) * 16 * cf.bn * 4;
}
int64_t workspace_bytes(const CfgEntry& cf, int64_t split, int64_t m, int64_t n) {
  if (split <= 1 || cf.kind == 3) return 0;
  const int64_t tiles = ((n + cf.bn - 1) / cf.bn) * ((m + cf.bm - 1) / cf.bm);
  return split * tiles * tile_partial_bytes(cf);
}
bool workspace_fits(const CfgEntry& cf, int64_t split, int64_t m, int64_t n) {
  if (split <= 1 || cf.kind == 3) return true;
  const int64_t tiles = ((n + cf.bn - 1) / cf.bn) * ((m + cf.bm - 1) / cf.bm);
  return tiles <= INFEROP_SPLITK_WS_COUNTERS &&
         workspace_bytes(cf, split, m, n) <= (int64_t)INFEROP_SPLITK_WS_BYTES;
}

// Compute units of the current device (cached per device ordinal).
hipError_t device_cus(int* cus) {
  static std::atomic<int> cached[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev >= 0 && dev < 64 && cached[dev].load(std::memory_order_relaxed) > 0) {
    *cus = cached[dev].load(std::memory_order_relaxed);
    return hipSuccess;
  }
  int v = 0;
  e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  if (v <= 0) return hipErrorInvalidDevice;
  if (dev >= 0 && dev < 64) cached[dev].store(v, std::memory_order_relaxed);
  *cus = v;
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
  info->waves = kCfgs[cfg].waves;
  info->kind = kCfgs[cfg].kind;
  info->name = kCfgs[cfg].name;
  info->grouped = ((kCfgs[cfg].kind == 2 || kCfgs[cfg].kind == 3) && kCfgs[cfg].fn_alt[0]) ||
                  (kCfgs[cfg].kind == 4 && kCfgs[cfg].fn_grp[0]);
  return hipSuccess;
}

extern "C" int64_t inferop_hip_gemm_workspace_bytes(int32_t cfg, int32_t split, int64_t m,
                                                    int64_t n, int64_t k) {
  if (cfg < 0 || cfg >= kNumCfgs || m <= 0 || n <= 0 || k < 128) return -1;
  int64_t s = split < 1 ? 1 : split;
  if (s > k / 128) s = k / 128;
  const CfgEntry& cf = kCfgs[cfg];
  if (cf.kind == 3) {
    int cus = 0;
    if (device_cus(&cus) != hipSuccess) cus = 256;
    const int64_t tiles = ((n + cf.bn - 1) / cf.bn) * ((m + cf.bm - 1) / cf.bm);
    return persist_plan(cf, tiles, k / 128, split, cus).ws_bytes;
  }
  const int64_t tiles = ((n + cf.bn - 1) / cf.bn) * ((m + cf.bm - 1) / cf.bm);
  if (s > 1 && cf.kind != 3 && tiles > INFEROP_SPLITK_WS_COUNTERS) return -1;
  return workspace_bytes(cf, s, m, n);
}

extern "C" int inferop_hip_splitk_reserve(void* stream) {
  float* ws = nullptr;
  int* cnt = nullptr;
  return get_workspace(static_cast<hipStream_t>(stream), &ws, &cnt);
}

extern "C" int inferop_hip_splitk_slots_used(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -1;
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  return g_ws[dev].used;
}

namespace inferop_hip {
namespace {
// Split-K partials and counters for a launch: the stream's workspace, or with
// noalloc the file-scope scratch.
hipError_t splitk_buffers(bool noalloc, hipStream_t st, float** ws, int** cnt) {
  return noalloc ? get_scratch(st, ws, cnt) : get_workspace(st, ws, cnt);
}

int gemm_block(void* c, const uint8_t* a_q, const float* a_scales, const uint8_t* b_q,
               const float* b_scales, int64_t m, int64_t n, int64_t k, int32_t out_dt,
               const inferop_gemm_launch* launch, void* stream, bool noalloc) {
  const int di = dt_index(out_dt);
  if (di < 0 || !launch || launch->cfg < 0 || launch->cfg >= kNumCfgs) return hipErrorInvalidValue;
  if (m <= 0 || n <= 0 || k <= 0 || k % 128 != 0) return hipErrorInvalidValue;
  if (m > 0x7FFFFFFF || n > 0x7FFFFFFF || k > 0x7FFFFFFF) return hipErrorInvalidValue;
  const CfgEntry& cf = kCfgs[launch->cfg];
  const int kg = (int)(k / 128);
  const int64_t tn = (n + cf.bn - 1) / cf.bn;
  const int64_t tm = (m + cf.bm - 1) / cf.bm;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int out_bytes = out_dt == kFp32 ? 4 : 2;
  const int vec_ok = (n % 4 == 0) && ((uintptr_t)c % (size_t)(4 * out_bytes) == 0);
  GemmArgs args{c,       a_q,    a_scales, b_q,    b_scales, nullptr,
                nullptr, (int)m, (int)n,   (int)k, vec_ok};
  if (cf.kind == 1) {
    // a stripe's 16 rows are addressed with 32-bit offsets
    if (16 * k > 0x7FFFFFFF) return hipErrorInvalidValue;
    int split = launch->split_k < 1 ? 1 : launch->split_k;
    if (split > kg) split = kg;
    if (tn > 0x7FFFFFFF || split > 65535 || tm > 65535) return hipErrorInvalidConfiguration;
    if (!workspace_fits(cf, split, m, n)) return hipErrorInvalidValue;
    if (split > 1) {
      hipError_t e = splitk_buffers(noalloc, st, &args.ws, &args.counters);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(cf.fn[di], dim3((unsigned)tn, (unsigned)split, (unsigned)tm),
                       dim3(64 * cf.waves), 0, st, args);
  } else if (cf.kind == 4) {
    // one workgroup per bn-row weight stripe group and 16*MT activation rows
    // over the whole K range, or over one of split_k K ranges (grid z, split-K
    // fixup); stripe and tile rows are addressed with 32-bit offsets.  The
    // scale preload holds wide_scale_cap() groups per wave; a longer range
    // per wave takes the kernel without it.
    if ((int64_t)cf.bm * k > 0x7FFFFFFF || (int64_t)cf.bn * k > 0x7FFFFFFF)
      return hipErrorInvalidValue;
    int split = launch->split_k < 1 ? 1 : launch->split_k;
    if (split > kg) split = kg;
    if (tn > 0x7FFFFFFF || tm > 65535 || split > 65535) return hipErrorInvalidConfiguration;
    if (!workspace_fits(cf, split, m, n)) return hipErrorInvalidValue;
    if (split > 1) {
      hipError_t e = splitk_buffers(noalloc, st, &args.ws, &args.counters);
      if (e != hipSuccess) return e;
    }
    const int64_t per_wave = ((kg + split - 1) / split + cf.waves - 1) / cf.waves;
    const KernelFn fn = per_wave <= wide_scale_cap() ? cf.fn[di] : cf.fn_alt[di];
    hipLaunchKernelGGL(fn, dim3((unsigned)tn, (unsigned)tm, (unsigned)split), dim3(64 * cf.waves),
                       0, st, args);
  } else if (cf.kind == 3) {
    // persistent: an even number of scale groups, one workgroup per CU (two
    // for 128x128 tiles, whose LDS allows it); split_k > 1 cuts the tiles of
    // the last, partial round into that many K ranges (fewer if the pieces
    // would not all run at once), added by the tail kernel afterwards
    const int64_t tiles = tn * tm;
    if (tiles > 0x7FFFFFFF || kg % 2 != 0) return hipErrorInvalidValue;
    if ((int64_t)(cf.bn > cf.bm ? cf.bn : cf.bm) * k > 0x7FFFFFFF) return hipErrorInvalidValue;
    int cus = 0;
    hipError_t e = device_cus(&cus);
    if (e != hipSuccess) return e;
    const PersistPlan pl = persist_plan(cf, tiles, kg, launch->split_k, cus);
    if (pl.split > 1) {
      if (pl.ws_bytes > (int64_t)INFEROP_SPLITK_WS_BYTES) return hipErrorInvalidValue;
      e = splitk_buffers(noalloc, st, &args.ws, &args.counters);
      if (e != hipSuccess) return e;
    }
    args.tail_split = pl.split;
    hipLaunchKernelGGL(cf.fn[di], dim3((unsigned)pl.grid), dim3(64 * cf.waves), 0, st, args);
    if (pl.split > 1) {
      e = hipGetLastError();
      if (e != hipSuccess) return e;
      const int64_t threads = pl.tail * (int64_t)cf.bn * cf.bm / 4;
      hipLaunchKernelGGL(cf.fn_tail[di], dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                         st, args, (int)(tiles - pl.tail), (int)pl.tail);
    }
  } else {
    const int64_t tiles = tn * tm;
    int split = launch->split_k < 1 ? 1 : launch->split_k;
    if (split > kg) split = kg;
    if (tiles > 0x7FFFFFFF || split > 65535) return hipErrorInvalidConfiguration;
    // tile rows are addressed with 32-bit buffer offsets
    if ((int64_t)(cf.bn > cf.bm ? cf.bn : cf.bm) * k > 0x7FFFFFFF) return hipErrorInvalidValue;
    if (!workspace_fits(cf, split, m, n)) return hipErrorInvalidValue;
    if (split > 1) {
      hipError_t e = splitk_buffers(noalloc, st, &args.ws, &args.counters);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(cf.fn[di], dim3((unsigned)tiles, (unsigned)split), dim3(64 * cf.waves), 0,
                       st, args);
  }
  return hipGetLastError();
}
}  // namespace
}  // namespace inferop_hip

extern "C" int inferop_hip_gemm_w8a8_block(void* c, const uint8_t* a_q, const float* a_scales,
                                           const uint8_t* b_q, const float* b_scales, int64_t m,
                                           int64_t n, int64_t k, int32_t out_dt,
                                           const inferop_gemm_launch* launch, void* stream) {
  return gemm_block(c, a_q, a_scales, b_q, b_scales, m, n, k, out_dt, launch, stream, false);
}

extern "C" int inferop_hip_gemm_w8a8_block_noalloc(void* c, const uint8_t* a_q,
                                                   const float* a_scales, const uint8_t* b_q,
                                                   const float* b_scales, int64_t m, int64_t n,
                                                   int64_t k, int32_t out_dt,
                                                   const inferop_gemm_launch* launch,
                                                   void* stream) {
  return gemm_block(c, a_q, a_scales, b_q, b_scales, m, n, k, out_dt, launch, stream, true);
}

namespace inferop_hip {
namespace {
template <int WK, int DT>
using QuantGemmFn = void (*)(GemmArgs, const void*, uint8_t*, float*);
template <int WK, int DT>
constexpr QuantGemmFn<WK, DT> kQuantGemm[3] = {gemm_quant_decode_kernel<WK, DT, kFp32>,
                                               gemm_quant_decode_kernel<WK, DT, kFp16>,
                                               gemm_quant_decode_kernel<WK, DT, kBf16>};
template <int WK>
void (*quant_gemm_fn(int32_t dt, int di))(GemmArgs, const void*, uint8_t*, float*) {
  switch (dt) {
    case kFp32: return kQuantGemm<WK, kFp32>[di];
    case kFp16: return kQuantGemm<WK, kFp16>[di];
    default: return kQuantGemm<WK, kBf16>[di];
  }
}
}  // namespace
}  // namespace inferop_hip

extern "C" int inferop_hip_quant_gemm_decode(void* c, uint8_t* q, float* qs, const void* x,
                                             int32_t dt, const uint8_t* b_q,
                                             const float* b_scales, int64_t m, int64_t n,
                                             int64_t k, int32_t out_dt, int32_t waves,
                                             void* stream) {
  const int di = dt_index(out_dt);
  if (di < 0 || (dt != kFp32 && dt != kFp16 && dt != kBf16)) return hipErrorInvalidValue;
  if (m < 1 || m > 8 || n <= 0 || k <= 0 || k % 128 != 0) return hipErrorInvalidValue;
  if (n > 0x7FFFFFFF || 16 * k > 0x7FFFFFFF) return hipErrorInvalidValue;
  if (waves != 4 && waves != 8) return hipErrorInvalidValue;
  if ((k / 128 + waves - 1) / waves > quant_gemm_cap()) return hipErrorInvalidValue;
  if ((uintptr_t)x % 16 != 0 || (uintptr_t)q % 8 != 0 || (uintptr_t)qs % 4 != 0)
    return hipErrorInvalidValue;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int out_bytes = out_dt == kFp32 ? 4 : 2;
  const int vec_ok = (n % 4 == 0) && ((uintptr_t)c % (size_t)(4 * out_bytes) == 0);
  GemmArgs args{c,       nullptr, nullptr, b_q,    b_scales, nullptr,
                nullptr, (int)m,  (int)n,  (int)k, vec_ok};
  const unsigned grid = (unsigned)((n + 15) / 16);
  if (waves == 8) {
    hipLaunchKernelGGL(quant_gemm_fn<8>(dt, di), dim3(grid), dim3(512), 0, st, args, x, q, qs);
  } else {
    hipLaunchKernelGGL(quant_gemm_fn<4>(dt, di), dim3(grid), dim3(256), 0, st, args, x, q, qs);
  }
  return hipGetLastError();
}

extern "C" int inferop_hip_gemm_w8a8_block_grouped(void* c, const uint8_t* a_q,
                                                   const float* a_scales, const uint8_t* b_q,
                                                   const float* b_scales, const int32_t* offsets,
                                                   int64_t m, int64_t n, int64_t k,
                                                   int64_t experts, int64_t max_m,
                                                   int32_t out_dt, int32_t cfg, void* stream) {
  const int di = dt_index(out_dt);
  if (di < 0 || cfg < 0 || cfg >= kNumCfgs) return hipErrorInvalidValue;
  const CfgEntry& cf = kCfgs[cfg];
  const bool grp_ok = ((cf.kind == 2 || cf.kind == 3) && cf.fn_alt[di]) ||
                      (cf.kind == 4 && cf.fn_grp[di] && cf.fn_grp_alt[di]);
  if (!grp_ok) return hipErrorInvalidValue;
  if (cf.kind == 3 && (k / 128) % 2 != 0) return hipErrorInvalidValue;
  if (m < 0 || n <= 0 || k <= 0 || k % 128 != 0 || experts <= 0 || max_m < 0)
    return hipErrorInvalidValue;
  // masked layout: m is the experts' max_m-row blocks end to end
  if (max_m > 0 && m != experts * max_m) return hipErrorInvalidValue;
  if (m == 0) return hipSuccess;
  if (m > 0x7FFFFFFF || n > 0x7FFFFFFF || k > 0x7FFFFFFF || experts > 0x7FFFFFFF)
    return hipErrorInvalidValue;
  // tile rows are addressed with 32-bit buffer offsets
  if ((int64_t)(cf.bn > cf.bm ? cf.bn : cf.bm) * k > 0x7FFFFFFF) return hipErrorInvalidValue;
  // every expert's M tiles fit in ceil(m / BM) + min(experts, m) virtual
  // tiles (an expert's last tile holds at least one of its rows; with
  // overlapping out-of-range offsets some tiles may fall outside the grid,
  // which leaves outputs unwritten but never addresses outside A, B or C)
  const int64_t tn = (n + cf.bn - 1) / cf.bn;
  const int64_t tmv = (m + cf.bm - 1) / cf.bm + (experts < m ? experts : m);
  if (tn * tmv > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int out_bytes = out_dt == kFp32 ? 4 : 2;
  const int vec_ok = (n % 4 == 0) && ((uintptr_t)c % (size_t)(4 * out_bytes) == 0);
  GemmArgs args{c,      a_q,    a_scales,     b_q,         b_scales,
                nullptr, nullptr, (int)m,     (int)n,      (int)k,
                vec_ok, offsets, (int)experts, (int)max_m};
  if (cf.kind == 4) {
    // one workgroup per (16-row weight stripe, virtual M tile of the experts)
    if (16 * k > 0x7FFFFFFF || tmv > 65535) return hipErrorInvalidConfiguration;
    const int64_t per_wave = (k / 128 + cf.waves - 1) / cf.waves;
    const KernelFn fn = per_wave <= wide_scale_cap() ? cf.fn_grp[di] : cf.fn_grp_alt[di];
    hipLaunchKernelGGL(fn, dim3((unsigned)tn, (unsigned)tmv), dim3(64 * cf.waves), 0, st, args);
    return hipGetLastError();
  }
  int64_t grid = tn * tmv;
  if (cf.kind == 3) {
    // persistent: one workgroup per CU (two for 128x128 tiles) walks the
    // tiles, whose number the kernel takes from the offsets
    int cus = 0;
    hipError_t e = device_cus(&cus);
    if (e != hipSuccess) return e;
    const int64_t slots = (int64_t)cus * (cf.bn * cf.bm <= 128 * 128 ? 2 : 1);
    if (grid > slots) grid = slots;
  }
  hipLaunchKernelGGL(cf.fn_alt[di], dim3((unsigned)grid, 1u), dim3(64 * cf.waves), 0, st, args);
  return hipGetLastError();
}
