// C++ front end of libinferop: the drop-in ops.h API and its C-ABI twin.
//
// Built with g++ and no HIP headers.  It owns what the reference keeps in
// kernels/api.cu and the *_impl functions (argument guards, dtype switch,
// device introspection) and the gfx950 tile selection that replaces the
// reference's SM-version switch (kernels/gemm/w8a8_block_fp8.cu:142-159).
// Kernels are reached through the thin C launch layer in hip_launch.h.
#include <cstdio>
#include <cstring>
#include <mutex>

#include "hip_launch.h"
#include "inferop/inferop_c.h"
#include "inferop/ops.h"

namespace inferop {
namespace {

// ---- device table (reference api.cu:12-34, made thread-safe) ---------------
constexpr int kMaxDevices = 64;

struct DeviceEntry {
  std::once_flag once;
  bool ok = false;
  int arch = -1;
  int cus = 0;
  char name[128] = "-";
};

struct DeviceTable {
  std::once_flag once;
  int count = 0;
  DeviceEntry dev[kMaxDevices];
};

DeviceTable& table() {
  static DeviceTable t;
  std::call_once(t.once, [] { t.count = inferop_hip_device_count(); });
  return t;
}

const DeviceEntry* device(int ordinal) {
  DeviceTable& t = table();
  if (ordinal < 0 || ordinal >= t.count || ordinal >= kMaxDevices) return nullptr;
  DeviceEntry& d = t.dev[ordinal];
  std::call_once(d.once, [&] {
    d.ok = inferop_hip_device_info(ordinal, d.name, sizeof(d.name), &d.arch, &d.cus) == 0;
    if (!d.ok) std::snprintf(d.name, sizeof(d.name), "-");
  });
  return d.ok ? &d : nullptr;
}

const DeviceEntry* current_device() {
  int ord = 0;
  if (inferop_hip_current_device(&ord) != 0) return nullptr;
  return device(ord);
}

bool valid_input_dtype(int32_t dt) { return dt == 0 || dt == 1 || dt == 2; }

int status_of_hip(int e) { return e == 0 ? INFEROP_OK : INFEROP_ERR_LAUNCH; }

// ---- gfx950 tile selection ----------------------------------------------------
// Kernel table indices (inferop_amd/csrc/gemm.hip, kCfgs).
enum GemmCfg : int32_t {
  kDecM16K1 = 0,
  kDecM16K2 = 1,
  kDecM16K4 = 2,
  kDecM16K8 = 3,
  kDecM32K4 = 4,
  kDecM64K4 = 5,
  kPreN256M128S3 = 6,
  kPreN128M256S3 = 7,
  kPreN128M128S2 = 8,
  kPreN128M128S4 = 9,
  kPreN256M256S2 = 10,
  kPreN128M64S4 = 11,
  kPreN128M32S4 = 12,
  kPreN128M16S4 = 13,
  kPreN64M64S4 = 14,
  kPreN128M64S3 = 15,
  kDecLdsK2 = 16,
  kDecLdsK4 = 17,
  kDecLdsK8 = 18,
  kPerN256M256 = 19,
  kPerN256M128 = 20,
  kPerN128M128 = 21,
  kDwM64K4 = 22,
  kDwM64K2 = 23,
  kDwM32K4 = 24,
  kDwM16K2 = 25,
  kDwM16K8 = 26,
  kDwM16K4 = 27,
  kDwM16K8W2 = 28,
  kDwN64M64 = 29,
  kDwN32M64 = 30,
  kDwN64M32 = 31,
  kDwN32M16 = 32,
  kDwN32M32 = 33,
  kDwM8K8 = 34,
  kDwM8K4 = 35,
};

struct GemmChoice {
  int32_t cfg;
  int32_t split;
};

GemmChoice select_gemm(int64_t m, int64_t n, int64_t k, int cus) {
  if (cus <= 0) cus = 256;
  const int64_t kg = k / 128;
  // The prefill kernels address a tile's rows with 32-bit offsets (256 rows
  // x K bytes); a K beyond that runs on the decode kernels at any M.
  const bool huge_k = k * 256 > 0x7FFFFFFF;
  // K split for the LDS-staged small tiles: as many splits as keep every
  // workgroup resident at two per CU (a second partial round costs more than
  // the splits gain), each split keeping at least four scale groups.
  auto small_tile_split = [&](int64_t tiles) {
    int64_t split = 2 * cus / tiles;
    if (split > kg / 4) split = kg / 4;
    return split < 1 ? int64_t(1) : split;
  };
  const int64_t stripes = (n + 15) / 16;  // 16-row weight stripes
  // Multi-stripe wide decode tiles: a workgroup owns 32 or 64 weight rows and
  // 32 or 64 activation rows, so a CU reads the activations once per 32-64
  // weight rows; K is split so that about one workgroup runs per CU (at least
  // 8 scale groups per split).  Two activation tiles of one row group share
  // the weight rows through L2 only when their workgroups land on the same
  // XCD (row groups a multiple of 8 along N), else one 64-row activation tile.
  const int64_t tx64 = (n + 63) / 64, tx32 = (n + 31) / 32;
  auto nt_split = [&](int64_t tiles) {
    int64_t sp = cus / tiles;
    if (sp > kg / 8) sp = kg / 8;
    return int32_t(sp < 1 ? 1 : sp);
  };
  // The 64-weight-row wide decode tiles from 65 to 512 rows: 32-row activation
  // tiles, else 64-row ones, each when one round of them (K split as above)
  // covers three quarters of the CUs.  From 96 scale groups up the K must be
  // split at least twice (one workgroup streaming the whole K is slower than
  // the persistent 128x128 tiles: M=128, N=7168, K=18432 61.0 us against 50.9;
  // at K=8192, M=160, N=4096 unsplit 64-row tiles take 23.5 us, 64x64
  // LDS-staged tiles 28.6), and unsplit 32-row tiles give way to 64-row tiles
  // that fill the CUs (M=96, N=4096, K=7168: 16.1 us against 15.7 in two;
  // M=224, N=2048, K=10240 22.8 against 18.6), except up to 32 scale groups,
  // where the split's partial round trip costs more than idle CUs and unsplit
  // 32-row tiles filling five eighths of them win (M=144, N=2048, K=4096: 10.0
  // us against 11.2 on 64-row tiles in two).  Every XCD reads all activation
  // rows, so M x K must fit its 4 MB L2 (M=448, N=2048, K=10240: 33.8 us
  // against 27.1 on 64x64 LDS-staged tiles).  Weight row groups that are not a
  // multiple of 8 put the activation tiles of a row group on different XCDs,
  // each reading the rows from HBM: then only a small weight (N <= 1024) over
  // at most six 32-row tiles, two thirds of the CUs busy (M=96, N=576, K=7168:
  // 8.9 us against 13.9 on 64x64 LDS-staged tiles).
  auto wide_tiles = [&](GemmChoice* ch) {
    if (kg < 8 || m * k > (int64_t(4) << 20)) return false;
    const bool aligned = tx64 % 8 == 0;
    if (!aligned && !(n <= 1024 && m <= 192)) return false;
    const int64_t w32 = tx64 * ((m + 31) / 32), w64 = tx64 * ((m + 63) / 64);
    const int32_t s32 = nt_split(w32), s64 = nt_split(w64);
    const int64_t c = cus;
    const bool fill32 = w32 <= c && (kg < 96 || s32 >= 2) &&
                        (!aligned   ? 3 * w32 * s32 >= 2 * c
                         : kg <= 32 ? 8 * w32 * s32 >= 5 * c
                                    : 4 * w32 * s32 >= 3 * c);
    const bool fill64 = aligned && w64 <= c && (kg >= 96 ? s64 >= 2 : 4 * w64 * s64 >= 3 * c);
    if (fill32 && (s32 >= 2 || kg <= 32 || !fill64)) {
      *ch = {kDwN64M32, s32};
      return true;
    }
    if (fill64) {
      *ch = {kDwN64M64, s64};
      return true;
    }
    return false;
  };
  // K split of the 64x64 LDS-staged tiles: unsplit below 32 scale groups,
  // else the split that keeps them to one round of two per CU, at most 6
  // (M=96, N=576, K=7168: 14 splits 13.9 us, 6 splits 11.4) and with the
  // fp32 partials of all splits, 4 * split * M bytes a column, no more than
  // the K bytes of weight a column (M=384, N=576, K=7168: 4 splits 13.6 us,
  // 6 splits 14.5).
  auto lds64_split = [&](int64_t t64) {
    if (kg < 32) return int32_t(1);
    int64_t split = small_tile_split(t64);
    if (split > 6) split = 6;
    if (4 * split * m > k) split = k / (4 * m);
    return int32_t(split < 1 ? 1 : split);
  };
  if (m > 32 && m <= 64 && !huge_k) {
    // one round of workgroups at most (one per CU); M=64, K=7168: N=4096
    // 14.0 -> 12.3 us (64x32 tiles, split 2), N=2112 12.3 -> 10.3 us (32x64,
    // split 3); K=2048, N=7168: 8.8 -> 7.4 us.  From 64 scale groups up only
    // with K split (M=48, N=7168, K=18432: 49.6 us unsplit, 35.5 on 128x64
    // LDS-staged tiles in four)
    // Up to 48 rows one 64-row activation tile (32x64 tiles) rather than
    // two 32-row tiles, the second not half full (M=40, N=4096, K=7168: 13.2
    // -> 11.5 us; N=7168, K=4096 12.1 -> 10.5).
    const int64_t w32 = tx64 * ((m + 31) / 32);
    if (m <= 48 && tx32 <= cus && (kg < 64 || nt_split(tx32) >= 2))
      return {kDwN32M64, nt_split(tx32)};
    if (tx64 % 8 == 0 && w32 <= cus && (kg < 64 || nt_split(w32) >= 2))
      return {kDwN64M32, nt_split(w32)};
    if (tx64 % 8 != 0 && tx32 <= cus) return {kDwN32M64, nt_split(tx32)};
  }
  if (m > 64 && m <= 128 && !huge_k && kg <= 16 && tx64 % 8 == 0) {
    // short K: one workgroup per 64 weight rows and 32 (or 64) activation rows
    // (M=128, N=4096, K=512: 4.9 -> 4.4 us; N=7168, K=2048: 11.6 -> 10.3 us)
    if (tx64 * ((m + 31) / 32) <= cus) return {kDwN64M32, 1};
    if (tx64 * ((m + 63) / 64) <= cus) return {kDwN64M64, 1};
  }
  if (m > 16 && m <= 64 && !huge_k) {
    // HBM-bound.  The wide decode kernel gives a workgroup one weight stripe
    // over the whole K range with the activation tiles of all M rows (no
    // split-K); the activations, which every stripe reads again from L2, are
    // what limits it, so it serves up to about one stripe per CU for a long K
    // and two for K <= 4096 (the configurations fit two workgroups per CU).
    if (m <= 32) {
      // 17 to 32 rows, from 32 scale groups up: 64x32 wide decode tiles, K
      // split to fill one round (M=24, K=7168: N=4096 11.6 -> 10.4 us, N=4608
      // 15.7 -> 11.2, N=36864 65.9 -> 55.1; N=7168, K=18432 46.0 -> 28.1).
      // Below that the stripe kernel, or 64x64 LDS-staged tiles beyond two
      // stripes per CU (N=24576, K=1536 15.0 -> 12.0; N=32768, K=512 11.3 ->
      // 6.8).
      if (kg >= 32) return {kDwN64M32, nt_split(tx64)};
      if (stripes > 2 * cus) return {kPreN64M64S4, 1};
      return {kDwM32K4, 1};
    }
    if (stripes <= cus && kg >= 32) {
      // with a quarter of the CUs or more left without a stripe, 128x32
      // tiles with K split across all CUs do better
      if (4 * stripes <= 3 * cus) {
        const int64_t tiles = ((n + 127) / 128) * ((m + 31) / 32);
        int64_t split = cus / tiles;
        if (split > kg / 4) split = kg / 4;
        return {kPreN128M32S4, int32_t(split < 1 ? 1 : split)};
      }
      return {kDwM64K4, 1};
    }
    if (stripes <= 2 * cus && kg >= 8 && kg <= 32) return {kDwM64K2, 1};
    // Beyond that, 128x64 tiles (a tile's activation rows are read once per
    // 128 weight rows); with a long K, split it so about two workgroups run
    // per CU (at most four splits: each split adds a partial round trip).
    const int64_t tiles = ((n + 127) / 128) * ((m + 63) / 64);
    int64_t split = 1;
    if (kg >= 32) {
      split = (2 * cus + tiles - 1) / tiles;
      if (split > 4) split = 4;
      if (split > kg / 4) split = kg / 4;
    }
    return {kPreN128M64S4, int32_t(split < 1 ? 1 : split)};
  }
  if (m > 64 && m <= 128 && !huge_k && ((n + 127) / 128) * ((m + 127) / 128) < cus) {
    // Multi-stripe wide decode tiles (64 weight rows x 64 activation rows,
    // the two activation tiles of a row group on one XCD) when they fill
    // three quarters of the CUs in one round below 64 scale groups, or split
    // K at least twice from 64 groups up (a CU then reads no more than on the
    // persistent 128x128 tiles with their 4-way tail split).  Same box, us:
    // M=100, N=4096, K=7168 17.0 -> 15.3; M=128: N=4096, K=7168 20.0 -> 15.5;
    // N=7168, K=4096 20.3 -> 15.9; N=2048, K=4096 14.4 -> 10.2; N=4096,
    // K=16384 41.4 -> 29.2; M=96, N=7168, K=7168 25.6 -> 22.4.  Not taken:
    // M=72, N=4608 (144 workgroups: 21.5 against 17.7) and M=128, N=7168,
    // K=18432 (one split: 61.0 against 50.9).
    // (and 32-row activation tiles where they fill the CUs: M=72, N=4608,
    // K=7168 17.9 -> 16.3 us; M=96, N=1536 11.8 -> 9.9; N=1024 11.7 -> 8.9)
    GemmChoice wc;
    if (wide_tiles(&wc)) return wc;
    // Still HBM-bound and too few 128x128 tiles to occupy every CU.  A long K
    // (64 scale groups or more): 128x64 tiles, three stages, K split so about
    // two workgroups run per CU (M=128, N=7168, K=18432: 57 us against 67 us
    // on 64x64).  Otherwise 64x64 tiles with four LDS stages, which keep more
    // weight bytes in flight per CU, split only from 32 scale groups up
    // (K=2048: 11.5 us unsplit, 12.6 us in two).
    if (kg >= 64) {
      // an even number of groups: the persistent 128x128 tiles, whose tiles
      // (all in the first, partial round) are cut into four K ranges (M=128,
      // N=7168, K=18432: 58.0 -> 49.9 us)
      if (kg % 2 == 0) return {kPerN128M128, 4};
      const int64_t tiles = ((n + 127) / 128) * ((m + 63) / 64);
      int64_t split = 2 * cus / tiles;
      if (split > 4) split = 4;
      if (split > kg / 16) split = kg / 16;
      return {kPreN128M64S3, int32_t(split < 1 ? 1 : split)};
    }
    // (the 64x64 tiles in one round of two per CU; beyond that the 128x128
    // tiles below: M=96, N=24576, K=1536 15.9 us)
    const int64_t tiles = ((n + 63) / 64) * ((m + 63) / 64);
    if (tiles <= 2 * cus) return {kPreN64M64S4, lds64_split(tiles)};
  }
  if (m > 64 && m <= 128 && !huge_k && kg >= 48 && (n + 255) / 256 <= cus &&
      ((n + 127) / 128) * ((m + 127) / 128) >= cus) {
    // More 128x128 tiles than CUs, but the 256x128 tiles (all M rows with 256
    // weight rows) fit in one round: a CU then reads the activations once per
    // 256 weight rows instead of once per 128, and no partial second round
    // follows.  Same box, K=7168: M=128, N=36864 96.6 -> 89.3 us, N=33280
    // 95.1 -> 88.9 us, M=96 92.7 -> 88.6 us; for K <= 4096 the 128x128 tiles
    // stay ahead by about 2%.
    return {kPreN256M128S3, 1};
  }
  if (m <= 16 && !huge_k) {
    // HBM-bound: a workgroup owns 16 weight rows over the whole K range on
    // the wide decode kernel.  A long K over stripes for fewer than half the
    // CUs is split across workgroups on the LDS-staged decode kernel (at
    // least 32 scale groups per split).  Otherwise: K beyond 8192 on two
    // waves with eight-deep rings; a stripe per CU or fewer on eight waves
    // with three-deep rings (all CUs busy with one workgroup each); many
    // stripes on the configurations that fit two workgroups per CU (four
    // waves three deep, or eight waves two deep beyond two stripes per CU).
    if (2 * stripes <= cus && kg >= 64) {
      int64_t split = cus / stripes;
      if (split > kg / 32) split = kg / 32;
      return {kDecLdsK8, int32_t(split)};
    }
    if (kg > 64) return {kDwM16K2, 1};
    // M <= 8: 8-row activation tiles, one load per group instead of two
    // (M=1, K=7168: N=2112 6.81 -> 6.44 us; K=2048, N=7168 5.32 -> 5.07 us;
    // M=8, N=4096 8.02 -> 7.37 us), four groups in flight per wave
    if (m <= 8 && kg <= 16) return {kDwM8K4, 1};
    if (m <= 8 && stripes <= cus) return {kDwM8K8, 1};
    if (m <= 8 && stripes <= 2 * cus) return {kDwM8K4, 1};
    if (kg <= 16) return {kDwM16K4, 1};
    if (stripes <= cus) return {kDwM16K8, 1};
    return {stripes > 2 * cus ? kDwM16K8W2 : kDwM16K4, 1};
  }
  if (m <= 64 || huge_k) {
    // HBM-bound: a workgroup owns 16 weight rows; its WK waves split the
    // scale groups, each streaming at most U groups with all loads in flight.
    // K is split across workgroups only when WK * U groups do not cover it.
    int32_t cfg;
    int64_t per_wg;
    if (m <= 32) {
      cfg = kDecM32K4, per_wg = 4 * 4;
    } else {
      cfg = kDecM64K4, per_wg = 4 * 2;
    }
    int64_t split = (kg + per_wg - 1) / per_wg;
    if (split < 1) split = 1;
    return {cfg, int32_t(split)};
  }
  // MFMA-bound.  The 256x256 tiles run on the persistent kernel when K has
  // an even number of scale groups (it keeps the pipeline going across a
  // CU's tiles and drains their stores in the background); the tiles of its
  // last, partial round are cut along K into up to 8 pieces that run at once
  // (their partials added by a second kernel) when the round time saved,
  // kg * (1 - 1/S) group-rounds, exceeds the cost of writing and re-reading
  // tail * S partial tiles of 256 KB (at ~5 TB/s, ~0.026 group-rounds each)
  // plus ~2.4 group-rounds of fixed cost (a group-round of 256x256 tiles
  // takes ~2.05 us on 256 CUs).  Measured on MI355X: M=4096, N=4608,
  // K=7168 (288 tiles) 177 -> 138 us with S=8 (128x128 tiles: 161 us);
  // M=512, N=7168, K=18432 (56 tiles) 220 -> 89 us with S=4 (128x128: 115-132
  // us); M=8192, N=7168, K=2048 (896 tiles) 139 us unsplit, 143 us with S=2.
  const int64_t t256 = ((n + 255) / 256) * ((m + 255) / 256);
  const int64_t t128 = ((n + 127) / 128) * ((m + 127) / 128);
  auto tail_split = [&]() -> int32_t {
    const int64_t tail = t256 >= cus ? t256 % cus : t256;
    if (tail == 0) return 1;
    int64_t sp = cus / tail;
    if (sp > 8) sp = 8;
    if (sp > kg / 2) sp = kg / 2;
    if (sp < 2) return 1;
    const double saved = (double)kg * (1.0 - 1.0 / (double)sp);
    const double cost = (double)(tail * sp) * 0.0256 + 2.4;
    return saved > cost ? int32_t(sp) : 1;
  };
  // at least one whole round of 256x256 tiles, or a long K: the persistent
  // 256x256 tiles (M=512, N=7168, K=18432 and M=1024: 89 / 150 us against
  // 115-132 / 189 us on 128x128 tiles)
  if (kg % 2 == 0 && (t256 >= cus || kg >= 96)) return {kPerN256M256, tail_split()};
  if (m <= 512 && t128 < cus) {
    // Up to 512 rows with fewer 128x128 tiles than CUs the product is still
    // HBM-bound: the weight read decides, and the 128x128 tiles leave CUs
    // idle.  First the wide decode tiles where they fill one round; else the
    // 64x64 LDS-staged tiles where they fit one round (from 48 scale groups
    // up only where they fit one per CU); else, with an even number of 48
    // scale groups or more, the persistent 128x128 tiles with their tail
    // split (all tiles in one, partial round, cut in up to 8 K ranges: the
    // fp32 partial round trip pays off only over a long K, at K=4096 it
    // loses 27.6 against 19.0 us); else the 128x128 tiles, split so that
    // the fp32 partials of all splits (4 * split * M bytes a column) stay
    // within half the weight bytes (M=448, N=6144, K=4096: 35.5 us in two,
    // 26.5 unsplit).  Same box, us (before: 128x128 tiles, K split in 3):
    // M=160, N=1536, K=7168 32.4 -> 11.1; M=192, N=4096, K=7168 35.8 ->
    // 21.2; N=576 31.5 -> 11.2; N=2112 32.2 -> 15.8; N=7168, K=2048 15.6 ->
    // 12.3; N=3072, K=1536 12.7 -> 8.6; M=256, N=4608, K=7168 36.9 -> 29.8;
    // M=384, N=4096, K=7168 44.9 -> 34.4; N=1536 33.6 -> 17.4; N=4096, K=512
    // 7.0 -> 5.9; M=160, N=6144, K=4096 27.6 (128x128, tail split) -> 19.0.
    GemmChoice wc;
    if (wide_tiles(&wc)) return wc;
    const int64_t t64 = ((n + 63) / 64) * ((m + 63) / 64);
    if (t64 <= cus || (kg < 48 && t64 <= 2 * cus)) return {kPreN64M64S4, lds64_split(t64)};
    if (kg % 2 == 0 && kg >= 48) return {kPerN128M128, 8};
    int64_t split = (cus + t128 - 1) / t128;
    if (split > 4) split = 4;
    if (split > kg / 16) split = kg / 16;
    while (split > 1 && 8 * split * m > k) --split;
    return {kPreN128M128S2, int32_t(split < 1 ? 1 : split)};
  }
  // Up to 256 rows (one 256-row tile) and 48 scale groups or more, with as
  // many 128x128 tiles as CUs or more: the persistent 256x256 tiles with
  // their tail split (M=160, N=18432, K=7168 65.6 -> 61.0 us; M=224 74.3 ->
  // 63.1)
  if (m <= 256 && kg % 2 == 0 && kg >= 48) return {kPerN256M256, tail_split()};
  // Otherwise: a 256x256 tile runs alone on a CU and does four 128x128 tiles'
  // work in about 1.5x their time (two 128x128 tiles share a CU); count whole
  // rounds of workgroups for both and take the cheaper one.
  const int64_t r256 = (t256 + cus - 1) / cus;
  const int64_t r128 = (t128 + 2 * cus - 1) / (2 * cus);
  if (2 * r256 * 3 < 2 * 2 * r128)
    return kg % 2 == 0 ? GemmChoice{kPerN256M256, tail_split()} : GemmChoice{kPreN256M256S2, 1};
  // Fewer 256x256 tiles than CUs but at least as many 128x128 tiles (so the
  // 128x128 tiles run unsplit, some CUs holding two), over a K of 48 scale
  // groups or more: the persistent 256x256 tiles, all in their first, partial
  // round and cut along K, read a quarter fewer operand bytes per CU
  // (configs[4] M=1000, N=4672, K=7168: 76 tiles cut in 3, 68.2 -> 59.5 us;
  // the 128x128 tiles put two on 40 CUs)
  if (kg % 2 == 0 && kg >= 48 && t256 < cus && t128 >= cus) {
    const int32_t s = tail_split();
    if (s >= 2) return {kPerN256M256, s};
  }
  // too few 128x128 tiles to fill the CUs: split K across workgroups, each
  // split keeping at least 16 scale groups (below that the fp32 partial
  // round trip costs more than the idle CUs) and at most four splits.
  int64_t split = 1;
  if (t128 < cus) {
    split = (cus + t128 - 1) / t128;
    int64_t max_split = kg / 16;
    if (max_split > 4) max_split = 4;
    if (split > max_split) split = max_split;
    if (split < 1) split = 1;
  }
  return {kPreN128M128S2, int32_t(split)};
}

// The automatic choice with its K split reduced, where needed, to what one
// split-K workspace slot holds (a long K on the decode kernels would otherwise
// ask for one partial tile per few groups).
GemmChoice choose_gemm(int64_t m, int64_t n, int64_t k, int cus) {
  GemmChoice ch = select_gemm(m, n, k, cus);
  while (ch.split > 1) {
    const int64_t b = inferop_hip_gemm_workspace_bytes(ch.cfg, ch.split, m, n, k);
    if (b >= 0 && b <= INFEROP_SPLITK_WS_BYTES) break;
    const int64_t s = b < 0 ? 1 : (int64_t)ch.split * INFEROP_SPLITK_WS_BYTES / b;
    ch.split = int32_t(s < ch.split ? (s < 1 ? 1 : s) : ch.split - 1);
  }
  return ch;
}

// The choice for a launch on `stream`: a split that needs workspace takes the
// stream's slot (its first split-K call allocates it); when the device has no
// slot left for this stream, the same configuration runs unsplit.
GemmChoice choose_gemm_on(int64_t m, int64_t n, int64_t k, int cus, void* stream) {
  GemmChoice ch = choose_gemm(m, n, k, cus);
  if (ch.split > 1 && inferop_hip_gemm_workspace_bytes(ch.cfg, ch.split, m, n, k) > 0 &&
      inferop_hip_splitk_reserve(stream) != 0)
    ch.split = 1;
  return ch;
}

// ---- implementations shared by the C++ and C entry points --------------------
int quant_impl(void* q, void* scales, const void* x, int32_t dt, int64_t rows, int64_t cols,
               int32_t group_size, void* stream) {
  // reference quant.cu:52 guard, then the dtype switch of quant.cu:56-74.
  if (rows <= 0 || cols <= 0 || group_size <= 0 || cols % group_size != 0) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(dt)) return INFEROP_ERR_DTYPE;
  if (!current_device()) return INFEROP_ERR_DEVICE;
  return status_of_hip(inferop_hip_quant_fp8_group(q, static_cast<float*>(scales), x, dt, rows, cols,
                                                   group_size, stream));
}

int dequant_impl(void* x, int32_t dt, const void* q, const void* scales, int64_t rows,
                 int64_t cols, int32_t group_size, void* stream) {
  // reference quant.cu:79 guard and quant.cu:84-102 dtype switch.
  if (rows <= 0 || cols <= 0 || group_size <= 0 || cols % group_size != 0) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(dt)) return INFEROP_ERR_DTYPE;
  if (!current_device()) return INFEROP_ERR_DEVICE;
  return status_of_hip(inferop_hip_dequant_fp8_group(x, dt, static_cast<const uint8_t*>(q),
                                                     static_cast<const float*>(scales), rows, cols,
                                                     group_size, stream));
}

int weight_quant_impl(void* b_q, void* b_scales, const void* w, int32_t dt, int64_t n, int64_t k,
                      int32_t group_size, int32_t block_n, void* stream) {
  if (group_size != 128 || block_n != 128 || n <= 0 || k <= 0 || k % 128 != 0)
    return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(dt)) return INFEROP_ERR_DTYPE;
  if (reinterpret_cast<uintptr_t>(w) % 16 != 0 || reinterpret_cast<uintptr_t>(b_q) % 8 != 0 ||
      reinterpret_cast<uintptr_t>(b_scales) % 4 != 0)
    return INFEROP_ERR_ARGUMENT;
  if (!current_device()) return INFEROP_ERR_DEVICE;
  return status_of_hip(inferop_hip_weight_block_quant(static_cast<uint8_t*>(b_q),
                                                      static_cast<float*>(b_scales), w, dt, n, k,
                                                      stream));
}

bool aligned(const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

int silu_quant_impl(void* q, void* scales, const void* gate_up, int32_t dt, int64_t tokens,
                    int64_t d, int32_t group_size, void* stream) {
  if (group_size != 128 || tokens <= 0 || d <= 0 || d % 128 != 0) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(dt)) return INFEROP_ERR_DTYPE;
  if (!aligned(gate_up, 16) || !aligned(q, 8) || !aligned(scales, 4)) return INFEROP_ERR_ARGUMENT;
  if (!current_device()) return INFEROP_ERR_DEVICE;
  return status_of_hip(inferop_hip_silu_mul_quant(static_cast<uint8_t*>(q),
                                                  static_cast<float*>(scales), gate_up, dt, tokens,
                                                  d, stream));
}

int rmsnorm_quant_impl(void* residual, void* q, void* scales, const void* x, const void* weight,
                       int32_t dt, int64_t rows, int64_t cols, float eps, int32_t group_size,
                       void* stream) {
  if (group_size != 128 || rows <= 0 || cols <= 0 || cols % 128 != 0) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(dt)) return INFEROP_ERR_DTYPE;
  if (!aligned(residual, 16) || !aligned(x, 16) || !aligned(weight, 16) || !aligned(q, 8) ||
      !aligned(scales, 4))
    return INFEROP_ERR_ARGUMENT;
  if (!current_device()) return INFEROP_ERR_DEVICE;
  return status_of_hip(inferop_hip_add_rmsnorm_quant(residual, static_cast<uint8_t*>(q),
                                                     static_cast<float*>(scales), x, weight, dt,
                                                     rows, cols, eps, stream));
}

int topk_impl(int32_t* ids, void* weights, const void* logits, int32_t tokens, int32_t experts,
              int32_t topk, int32_t renormalize, void* stream) {
  // reference moe/topk_softmax.cu:89-92 guard
  if (tokens <= 0 || experts <= 0 || experts > 1024 || topk <= 0 || topk > experts)
    return INFEROP_ERR_SHAPE;
  if (!current_device()) return INFEROP_ERR_DEVICE;
  return status_of_hip(inferop_hip_topk_softmax(ids, static_cast<float*>(weights),
                                                static_cast<const float*>(logits), tokens, experts,
                                                topk, renormalize ? 1 : 0, stream));
}

bool gemm_shape_ok(int64_t m, int64_t n, int64_t k, int32_t group_size, int32_t block_n) {
  // reference w8a8_block_fp8.cu:167-173, including its diagnostic line.
  if (group_size != 128 || block_n != 128 || k % 128 != 0 || m <= 0 || n <= 0) {
    std::fprintf(stderr,
                 "[inferop] w8a8_block_fp8_gemm: unsupported shape (m=%lld n=%lld k=%lld gs=%d "
                 "bn=%d); v0.1 requires gs=bn=128, k%%128==0\n",
                 (long long)m, (long long)n, (long long)k, group_size, block_n);
    return false;
  }
  return true;
}

const DeviceEntry* gemm_device() {
  const DeviceEntry* d = current_device();
  if (!d || d->arch != 0x950) {
    // The kernels are built for gfx950 only (arch parsed as hex digits: 0x950).
    static std::once_flag warned;
    std::call_once(warned, [] {
      std::fprintf(stderr, "[inferop] w8a8_block_fp8_gemm: current device is not gfx950\n");
    });
    return nullptr;
  }
  return d;
}

int gemm_launch(void* c, const void* a_q, const void* a_scales, const void* b_q,
                const void* b_scales, int64_t m, int64_t n, int64_t k, int32_t out_dt, int32_t cfg,
                int32_t split, void* stream) {
  inferop_gemm_launch l{cfg, split};
  return status_of_hip(inferop_hip_gemm_w8a8_block(
      c, static_cast<const uint8_t*>(a_q), static_cast<const float*>(a_scales),
      static_cast<const uint8_t*>(b_q), static_cast<const float*>(b_scales), m, n, k, out_dt, &l,
      stream));
}

int gemm_impl(void* c, const void* a_q, const void* a_scales, const void* b_q,
              const void* b_scales, int64_t m, int64_t n, int64_t k, int32_t group_size,
              int32_t block_n, int32_t out_dt, void* stream) {
  if (!gemm_shape_ok(m, n, k, group_size, block_n)) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(out_dt)) return INFEROP_ERR_DTYPE;  // reference :185-186 silent no-op
  const DeviceEntry* d = gemm_device();
  if (!d) return INFEROP_ERR_DEVICE;
  const GemmChoice ch = choose_gemm_on(m, n, k, d->cus, stream);
  return gemm_launch(c, a_q, a_scales, b_q, b_scales, m, n, k, out_dt, ch.cfg, ch.split, stream);
}

// The quantizer and the GEMM in one call (the decode step's pair).  Where the
// automatic GEMM choice is an unsplit 8-row wide decode configuration (M <= 8)
// and every wave of it takes at most 8 scale groups, one kernel quantizes the
// activations inside the GEMM; otherwise the quantizer and the GEMM run as two
// launches on the stream.  Either way q / scales are the quantizer's output
// and c the GEMM's with the automatic choice, bit for bit.
int quant_gemm_plan(int64_t m, int64_t k, const GemmChoice& ch) {
  if (m > 8 || ch.split != 1 || (ch.cfg != kDwM8K8 && ch.cfg != kDwM8K4)) return 0;
  const int waves = ch.cfg == kDwM8K8 ? 8 : 4;
  return (k / 128 + waves - 1) / waves <= 8 ? waves : 0;  // 8 groups per wave at most
}

int quant_gemm_impl(void* c, void* q, void* scales, const void* x, int32_t dt, const void* b_q,
                    const void* b_scales, int64_t m, int64_t n, int64_t k, int32_t group_size,
                    int32_t block_n, int32_t out_dt, void* stream) {
  if (!gemm_shape_ok(m, n, k, group_size, block_n)) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(dt) || !valid_input_dtype(out_dt)) return INFEROP_ERR_DTYPE;
  const DeviceEntry* d = gemm_device();
  if (!d) return INFEROP_ERR_DEVICE;
  const GemmChoice ch = choose_gemm_on(m, n, k, d->cus, stream);
  const int waves = quant_gemm_plan(m, k, ch);
  if (waves > 0 && aligned(x, 16) && aligned(q, 8) && aligned(scales, 4)) {
    return status_of_hip(inferop_hip_quant_gemm_decode(
        c, static_cast<uint8_t*>(q), static_cast<float*>(scales), x, dt,
        static_cast<const uint8_t*>(b_q), static_cast<const float*>(b_scales), m, n, k, out_dt,
        waves, stream));
  }
  const int st = status_of_hip(inferop_hip_quant_fp8_group(q, static_cast<float*>(scales), x, dt,
                                                           m, k, 128, stream));
  if (st != INFEROP_OK) return st;
  return gemm_launch(c, q, scales, b_q, b_scales, m, n, k, out_dt, ch.cfg, ch.split, stream);
}

// Grouped (MoE expert) GEMM: the configuration from the mean rows per expert.
// Up to 8 rows per expert (decode routings) the wide decode kernel: one
// workgroup per (16-row weight stripe, expert tile) streams the stripe over
// the whole K range, so the weights of every expert with rows leave HBM once
// at the decode kernel's rate (32 experts, N=4096, K=7168: 2 rows per expert
// 124 us vs 154 us on the persistent 128x128 tiles, 8 rows 165 vs 173 us; at
// 16 rows 243 vs 174 us).  Beyond that, with an even K / 128, the persistent
// kernels, whose load pipeline runs on
// across a workgroup's tiles, stream the experts' weights best whatever the
// rows: two 128x128 workgroups per CU below about 96 rows per expert, one
// 256x256 beyond (measured at 32 experts, N=4096, K=7168: 2 rows per expert
// 153 us on 128x128 vs 155 us on 16-row tiled; 32 rows 178 vs 217 us; 64 rows
// 191 us vs 239 us on 256x256; 128 rows 251 us on 256x256 vs 286 us on
// 128x128 and 385 us tiled; 512 rows 592 vs 843 us tiled).  With an odd
// K / 128 the tiled kernels: 16-row tiles below 16 rows per expert, 32-row
// below 24, 64-row three-stage below 64, 128x128 beyond.
// m: the rows the tile choice is made for (masked layout: the expected rows
// per expert times the experts); launch_m: the rows the grid is launched over
// (masked layout: experts * max_m), which the wide decode kernel's grid limit
// applies to.
int32_t select_grouped(int64_t m, int64_t launch_m, int64_t k, int64_t num_experts) {
  const int64_t avg = m / (num_experts > 0 ? num_experts : 1);
  const int64_t ne = num_experts < launch_m ? num_experts : launch_m;
  if (avg <= 8 && 16 * k <= 0x7FFFFFFF && (launch_m + 15) / 16 + ne <= 65535) return kDwM16K4;
  if ((k / 128) % 2 == 0) return avg < 96 ? kPerN128M128 : kPerN256M256;
  if (avg < 16) return kPreN128M16S4;
  if (avg < 24) return kPreN128M32S4;
  if (avg < 64) return kPreN128M64S3;
  return kPreN128M128S2;
}

bool grouped_shape_ok(int64_t m, int64_t n, int64_t k, int64_t experts, int32_t group_size,
                      int32_t block_n) {
  if (group_size != 128 || block_n != 128 || k <= 0 || k % 128 != 0 || m < 0 || n <= 0 ||
      experts <= 0 || experts > 0x7FFFFFFF) {
    std::fprintf(stderr,
                 "[inferop] w8a8_block_fp8_grouped_gemm: unsupported shape (m=%lld n=%lld k=%lld "
                 "experts=%lld gs=%d bn=%d); requires gs=bn=128, k%%128==0, experts>=1\n",
                 (long long)m, (long long)n, (long long)k, (long long)experts, group_size,
                 block_n);
    return false;
  }
  return true;
}

int grouped_launch(void* c, const void* a_q, const void* a_scales, const void* b_q,
                   const void* b_scales, const void* offsets, int64_t m, int64_t n, int64_t k,
                   int64_t experts, int64_t max_m, int32_t out_dt, int32_t cfg, void* stream) {
  return status_of_hip(inferop_hip_gemm_w8a8_block_grouped(
      c, static_cast<const uint8_t*>(a_q), static_cast<const float*>(a_scales),
      static_cast<const uint8_t*>(b_q), static_cast<const float*>(b_scales),
      static_cast<const int32_t*>(offsets), m, n, k, experts, max_m, out_dt, cfg, stream));
}

// Masked layout: experts x max_m rows (and C rows), counts on the device.
bool masked_shape_ok(int64_t max_m, int64_t n, int64_t k, int64_t experts, int32_t group_size,
                     int32_t block_n) {
  if (group_size != 128 || block_n != 128 || k <= 0 || k % 128 != 0 || max_m < 0 || n <= 0 ||
      experts <= 0 || experts > 0x7FFFFFFF || (max_m > 0 && experts > 0x7FFFFFFF / max_m)) {
    std::fprintf(stderr,
                 "[inferop] w8a8_block_fp8_grouped_gemm_masked: unsupported shape (max_m=%lld "
                 "n=%lld k=%lld experts=%lld gs=%d bn=%d); requires gs=bn=128, k%%128==0, "
                 "experts>=1, experts*max_m < 2^31\n",
                 (long long)max_m, (long long)n, (long long)k, (long long)experts, group_size,
                 block_n);
    return false;
  }
  return true;
}

int masked_impl(void* c, const void* a_q, const void* a_scales, const void* b_q,
                const void* b_scales, const void* masked_m, int64_t max_m, int64_t n, int64_t k,
                int64_t experts, int64_t expected_m, int32_t group_size, int32_t block_n,
                int32_t out_dt, int32_t cfg, void* stream) {
  if (!masked_shape_ok(max_m, n, k, experts, group_size, block_n)) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(out_dt)) return INFEROP_ERR_DTYPE;
  if (cfg < 0) {
    const int64_t rows = expected_m > 0 ? (expected_m < max_m ? expected_m : max_m) : max_m;
    cfg = select_grouped(rows * experts, experts * max_m, k, experts);
  }
  if (max_m == 0) return INFEROP_OK;
  if (!gemm_device()) return INFEROP_ERR_DEVICE;
  return grouped_launch(c, a_q, a_scales, b_q, b_scales, masked_m, experts * max_m, n, k,
                        experts, max_m, out_dt, cfg, stream);
}

int grouped_impl(void* c, const void* a_q, const void* a_scales, const void* b_q,
                 const void* b_scales, const void* offsets, int64_t m, int64_t n, int64_t k,
                 int64_t experts, int32_t group_size, int32_t block_n, int32_t out_dt,
                 void* stream) {
  if (!grouped_shape_ok(m, n, k, experts, group_size, block_n)) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(out_dt)) return INFEROP_ERR_DTYPE;
  if (m == 0) return INFEROP_OK;
  if (!gemm_device()) return INFEROP_ERR_DEVICE;
  return grouped_launch(c, a_q, a_scales, b_q, b_scales, offsets, m, n, k, experts, 0, out_dt,
                        select_grouped(m, m, k, experts), stream);
}

}  // namespace

// ---- ops.h --------------------------------------------------------------------
bool has_cuda() { return table().count > 0; }

int device_count() { return table().count; }

const char* device_name(int ordinal) {
  const DeviceEntry* d = device(ordinal);
  return d ? d->name : "-";
}

int device_sm_version(int ordinal) {
  const DeviceEntry* d = device(ordinal);
  if (!d || d->arch < 0) return -1;
  // arch holds the gfx digits read as hex (gfx950 -> 0x950); report them as
  // the decimal-looking number 950 (gfx90a -> 0x90a is reported as 2314).
  int v = d->arch;
  if (((v >> 8) & 0xF) <= 9 && ((v >> 4) & 0xF) <= 9 && (v & 0xF) <= 9)
    return ((v >> 8) & 0xF) * 100 + ((v >> 4) & 0xF) * 10 + (v & 0xF);
  return v;
}

void quant_fp8_per_token_group(void* q, void* scales, const void* x, dtype dt, int64_t rows,
                               int64_t cols, int group_size, void* stream) {
  (void)quant_impl(q, scales, x, int32_t(dt), rows, cols, group_size, stream);
}

void dequant_fp8_per_token_group(void* x, dtype dt, const void* q, const void* scales,
                                 int64_t rows, int64_t cols, int group_size, void* stream) {
  (void)dequant_impl(x, int32_t(dt), q, scales, rows, cols, group_size, stream);
}

void w8a8_block_fp8_gemm(void* c, const void* a_q, const void* a_scales, const void* b_q,
                         const void* b_scales, int64_t m, int64_t n, int64_t k, int group_size,
                         int block_n, dtype out_dt, void* stream) {
  (void)gemm_impl(c, a_q, a_scales, b_q, b_scales, m, n, k, group_size, block_n,
                  int32_t(out_dt), stream);
}

void quant_w8a8_block_fp8_gemm(void* c, void* q, void* scales, const void* x, dtype dt,
                               const void* b_q, const void* b_scales, int64_t m, int64_t n,
                               int64_t k, int group_size, int block_n, dtype out_dt,
                               void* stream) {
  (void)quant_gemm_impl(c, q, scales, x, int32_t(dt), b_q, b_scales, m, n, k, group_size, block_n,
                        int32_t(out_dt), stream);
}

void w8a8_block_fp8_grouped_gemm(void* c, const void* a_q, const void* a_scales,
                                 const void* b_q, const void* b_scales,
                                 const void* expert_offsets, int64_t m, int64_t n, int64_t k,
                                 int64_t num_experts, int group_size, int block_n, dtype out_dt,
                                 void* stream) {
  (void)grouped_impl(c, a_q, a_scales, b_q, b_scales, expert_offsets, m, n, k, num_experts,
                     group_size, block_n, int32_t(out_dt), stream);
}

void w8a8_block_fp8_grouped_gemm_masked(void* c, const void* a_q, const void* a_scales,
                                        const void* b_q, const void* b_scales,
                                        const void* masked_m, int64_t max_m, int64_t n, int64_t k,
                                        int64_t num_experts, int64_t expected_m, int group_size,
                                        int block_n, dtype out_dt, void* stream) {
  (void)masked_impl(c, a_q, a_scales, b_q, b_scales, masked_m, max_m, n, k, num_experts,
                    expected_m, group_size, block_n, int32_t(out_dt), -1, stream);
}

void topk_softmax(int32_t* topk_ids, void* topk_weights, const void* logits, int tokens,
                  int num_experts, int topk, bool renormalize, void* stream) {
  (void)topk_impl(topk_ids, topk_weights, logits, tokens, num_experts, topk, renormalize ? 1 : 0,
                  stream);
}

void quant_fp8_weight_block(void* b_q, void* b_scales, const void* w, dtype dt, int64_t n,
                            int64_t k, int group_size, int block_n, void* stream) {
  (void)weight_quant_impl(b_q, b_scales, w, int32_t(dt), n, k, group_size, block_n, stream);
}

void silu_and_mul_quant_fp8(void* q, void* scales, const void* gate_up, dtype dt, int64_t tokens,
                            int64_t d, int group_size, void* stream) {
  (void)silu_quant_impl(q, scales, gate_up, int32_t(dt), tokens, d, group_size, stream);
}

void fused_add_rmsnorm_quant_fp8(void* residual, void* q, void* scales, const void* x,
                                 const void* weight, dtype dt, int64_t rows, int64_t cols,
                                 float eps, int group_size, void* stream) {
  (void)rmsnorm_quant_impl(residual, q, scales, x, weight, int32_t(dt), rows, cols, eps,
                           group_size, stream);
}

}  // namespace inferop

// ---- inferop_c.h ------------------------------------------------------------------
using namespace inferop;

extern "C" const char* inferop_status_string(int status) {
  switch (status) {
    case INFEROP_OK: return "ok";
    case INFEROP_ERR_SHAPE: return "unsupported shape";
    case INFEROP_ERR_DTYPE: return "unsupported dtype";
    case INFEROP_ERR_DEVICE: return "no usable gfx950 device";
    case INFEROP_ERR_LAUNCH: return "HIP runtime error";
    case INFEROP_ERR_ARGUMENT: return "invalid argument";
  }
  return "unknown status";
}

extern "C" int inferop_has_device(void) { return has_cuda() ? 1 : 0; }
extern "C" int inferop_device_count(void) { return device_count(); }
extern "C" const char* inferop_device_name(int ordinal) { return device_name(ordinal); }
extern "C" int inferop_device_arch(int ordinal) { return device_sm_version(ordinal); }

extern "C" int inferop_quant_fp8_per_token_group(void* q, void* scales, const void* x, int32_t dt,
                                                 int64_t rows, int64_t cols, int32_t group_size,
                                                 void* stream) {
  return quant_impl(q, scales, x, dt, rows, cols, group_size, stream);
}

extern "C" int inferop_dequant_fp8_per_token_group(void* x, int32_t dt, const void* q,
                                                   const void* scales, int64_t rows, int64_t cols,
                                                   int32_t group_size, void* stream) {
  return dequant_impl(x, dt, q, scales, rows, cols, group_size, stream);
}

extern "C" int inferop_w8a8_block_fp8_gemm(void* c, const void* a_q, const void* a_scales,
                                           const void* b_q, const void* b_scales, int64_t m,
                                           int64_t n, int64_t k, int32_t group_size,
                                           int32_t block_n, int32_t out_dt, void* stream) {
  return gemm_impl(c, a_q, a_scales, b_q, b_scales, m, n, k, group_size, block_n, out_dt, stream);
}

extern "C" int inferop_quant_w8a8_block_fp8_gemm(void* c, void* q, void* scales, const void* x,
                                                 int32_t dt, const void* b_q, const void* b_scales,
                                                 int64_t m, int64_t n, int64_t k,
                                                 int32_t group_size, int32_t block_n,
                                                 int32_t out_dt, void* stream) {
  return quant_gemm_impl(c, q, scales, x, dt, b_q, b_scales, m, n, k, group_size, block_n, out_dt,
                         stream);
}

extern "C" int inferop_quant_w8a8_block_fp8_gemm_launches(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 128 != 0) return -1;
  const DeviceEntry* d = current_device();
  return quant_gemm_plan(m, k, choose_gemm(m, n, k, d ? d->cus : 256)) > 0 ? 1 : 2;
}

extern "C" int inferop_w8a8_block_fp8_gemm_noalloc(void* c, const void* a_q, const void* a_scales,
                                                   const void* b_q, const void* b_scales,
                                                   int64_t m, int64_t n, int64_t k,
                                                   int32_t group_size, int32_t block_n,
                                                   int32_t out_dt, void* stream) {
  // gemm_impl's guards and automatic choice; only the split-K buffers differ
  if (!gemm_shape_ok(m, n, k, group_size, block_n)) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(out_dt)) return INFEROP_ERR_DTYPE;
  const DeviceEntry* d = gemm_device();
  if (!d) return INFEROP_ERR_DEVICE;
  const GemmChoice ch = choose_gemm(m, n, k, d->cus);
  const int64_t need = inferop_hip_gemm_workspace_bytes(ch.cfg, ch.split, m, n, k);
  if (need < 0 || need > INFEROP_SPLITK_WS_BYTES) {
    std::fprintf(stderr,
                 "[inferop] w8a8_block_fp8_gemm_noalloc: shape (m=%lld n=%lld k=%lld) needs "
                 "%lld bytes of split-K scratch, more than the fixed %lld\n",
                 (long long)m, (long long)n, (long long)k, (long long)need,
                 (long long)INFEROP_SPLITK_WS_BYTES);
    return INFEROP_ERR_ARGUMENT;
  }
  inferop_gemm_launch l{ch.cfg, ch.split};
  return status_of_hip(inferop_hip_gemm_w8a8_block_noalloc(
      c, static_cast<const uint8_t*>(a_q), static_cast<const float*>(a_scales),
      static_cast<const uint8_t*>(b_q), static_cast<const float*>(b_scales), m, n, k, out_dt, &l,
      stream));
}

extern "C" int inferop_topk_softmax(int32_t* topk_ids, void* topk_weights, const void* logits,
                                    int32_t tokens, int32_t num_experts, int32_t topk,
                                    int32_t renormalize, void* stream) {
  return topk_impl(topk_ids, topk_weights, logits, tokens, num_experts, topk, renormalize, stream);
}

extern "C" int inferop_quant_fp8_weight_block(void* b_q, void* b_scales, const void* w, int32_t dt,
                                              int64_t n, int64_t k, int32_t group_size,
                                              int32_t block_n, void* stream) {
  return weight_quant_impl(b_q, b_scales, w, dt, n, k, group_size, block_n, stream);
}

extern "C" int inferop_silu_and_mul_quant_fp8(void* q, void* scales, const void* gate_up,
                                              int32_t dt, int64_t tokens, int64_t d,
                                              int32_t group_size, void* stream) {
  return silu_quant_impl(q, scales, gate_up, dt, tokens, d, group_size, stream);
}

extern "C" int inferop_fused_add_rmsnorm_quant_fp8(void* residual, void* q, void* scales,
                                                   const void* x, const void* weight, int32_t dt,
                                                   int64_t rows, int64_t cols, float eps,
                                                   int32_t group_size, void* stream) {
  return rmsnorm_quant_impl(residual, q, scales, x, weight, dt, rows, cols, eps, group_size,
                            stream);
}

extern "C" int inferop_gemm_num_configs(void) { return inferop_hip_gemm_num_configs(); }

extern "C" const char* inferop_gemm_config_name(int config) {
  inferop_gemm_cfg_info info;
  if (inferop_hip_gemm_config_info(config, &info) != 0) return "invalid";
  return info.name;
}

extern "C" int inferop_w8a8_block_fp8_gemm_config(void* c, const void* a_q, const void* a_scales,
                                                  const void* b_q, const void* b_scales, int64_t m,
                                                  int64_t n, int64_t k, int32_t out_dt,
                                                  int32_t config, int32_t split_k, void* stream) {
  if (!gemm_shape_ok(m, n, k, 128, 128)) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(out_dt)) return INFEROP_ERR_DTYPE;
  if (config < 0 || config >= inferop_hip_gemm_num_configs() || split_k < 1)
    return INFEROP_ERR_ARGUMENT;
  // the persistent kernels take an even number of scale groups
  inferop_gemm_cfg_info info{};
  if (inferop_hip_gemm_config_info(config, &info) != 0) return INFEROP_ERR_ARGUMENT;
  if (info.kind == 3 && (k / 128) % 2 != 0) return INFEROP_ERR_ARGUMENT;
  // the split-K workspace has a fixed capacity
  const int64_t ws = inferop_hip_gemm_workspace_bytes(config, split_k, m, n, k);
  if (ws < 0 || ws > INFEROP_SPLITK_WS_BYTES) return INFEROP_ERR_ARGUMENT;
  if (!gemm_device()) return INFEROP_ERR_DEVICE;
  // a split needs the stream's workspace slot; none left on the device for
  // this stream is an argument error (nothing is launched)
  if (ws > 0 && inferop_hip_splitk_reserve(stream) != 0) return INFEROP_ERR_ARGUMENT;
  return gemm_launch(c, a_q, a_scales, b_q, b_scales, m, n, k, out_dt, config, split_k, stream);
}

extern "C" int inferop_w8a8_block_fp8_grouped_gemm(void* c, const void* a_q, const void* a_scales,
                                                   const void* b_q, const void* b_scales,
                                                   const int32_t* expert_offsets, int64_t m,
                                                   int64_t n, int64_t k, int64_t num_experts,
                                                   int32_t group_size, int32_t block_n,
                                                   int32_t out_dt, void* stream) {
  return grouped_impl(c, a_q, a_scales, b_q, b_scales, expert_offsets, m, n, k, num_experts,
                      group_size, block_n, out_dt, stream);
}

extern "C" int inferop_w8a8_block_fp8_grouped_gemm_config(
    void* c, const void* a_q, const void* a_scales, const void* b_q, const void* b_scales,
    const int32_t* expert_offsets, int64_t m, int64_t n, int64_t k, int64_t num_experts,
    int32_t out_dt, int32_t config, void* stream) {
  if (!grouped_shape_ok(m, n, k, num_experts, 128, 128)) return INFEROP_ERR_SHAPE;
  if (!valid_input_dtype(out_dt)) return INFEROP_ERR_DTYPE;
  inferop_gemm_cfg_info info{};
  if (config < 0 || config >= inferop_hip_gemm_num_configs() ||
      inferop_hip_gemm_config_info(config, &info) != 0 || !info.grouped)
    return INFEROP_ERR_ARGUMENT;
  if (info.kind == 3 && (k / 128) % 2 != 0) return INFEROP_ERR_ARGUMENT;
  if (m == 0) return INFEROP_OK;
  if (!gemm_device()) return INFEROP_ERR_DEVICE;
  return grouped_launch(c, a_q, a_scales, b_q, b_scales, expert_offsets, m, n, k, num_experts, 0,
                        out_dt, config, stream);
}

extern "C" int inferop_w8a8_block_fp8_grouped_gemm_masked(
    void* c, const void* a_q, const void* a_scales, const void* b_q, const void* b_scales,
    const int32_t* masked_m, int64_t max_m, int64_t n, int64_t k, int64_t num_experts,
    int64_t expected_m, int32_t group_size, int32_t block_n, int32_t out_dt, void* stream) {
  return masked_impl(c, a_q, a_scales, b_q, b_scales, masked_m, max_m, n, k, num_experts,
                     expected_m, group_size, block_n, out_dt, -1, stream);
}

extern "C" int inferop_w8a8_block_fp8_grouped_gemm_masked_config(
    void* c, const void* a_q, const void* a_scales, const void* b_q, const void* b_scales,
    const int32_t* masked_m, int64_t max_m, int64_t n, int64_t k, int64_t num_experts,
    int32_t out_dt, int32_t config, void* stream) {
  inferop_gemm_cfg_info info{};
  if (config < 0 || config >= inferop_hip_gemm_num_configs() ||
      inferop_hip_gemm_config_info(config, &info) != 0 || !info.grouped)
    return INFEROP_ERR_ARGUMENT;
  if (info.kind == 3 && (k / 128) % 2 != 0) return INFEROP_ERR_ARGUMENT;
  return masked_impl(c, a_q, a_scales, b_q, b_scales, masked_m, max_m, n, k, num_experts, 0, 128,
                     128, out_dt, config, stream);
}

extern "C" int inferop_grouped_gemm_select(int64_t m, int64_t n, int64_t k, int64_t num_experts,
                                           int32_t* config) {
  if (m < 0 || n <= 0 || k <= 0 || k % 128 != 0 || num_experts <= 0 || !config)
    return INFEROP_ERR_ARGUMENT;
  *config = select_grouped(m, m, k, num_experts);
  return INFEROP_OK;
}

extern "C" int inferop_grouped_gemm_masked_select(int64_t max_m, int64_t n, int64_t k,
                                                  int64_t num_experts, int64_t expected_m,
                                                  int32_t* config) {
  if (max_m < 0 || n <= 0 || k <= 0 || k % 128 != 0 || num_experts <= 0 || !config ||
      (max_m > 0 && num_experts > 0x7FFFFFFF / max_m))
    return INFEROP_ERR_ARGUMENT;
  const int64_t rows = expected_m > 0 ? (expected_m < max_m ? expected_m : max_m) : max_m;
  *config = select_grouped(rows * num_experts, num_experts * max_m, k, num_experts);
  return INFEROP_OK;
}

extern "C" int inferop_splitk_workspace_info(int32_t* slots_used, int32_t* slots_total,
                                             int64_t* slot_bytes) {
  if (!current_device()) return INFEROP_ERR_DEVICE;
  const int used = inferop_hip_splitk_slots_used();
  if (used < 0) return INFEROP_ERR_LAUNCH;
  if (slots_used) *slots_used = used;
  if (slots_total) *slots_total = INFEROP_SPLITK_WS_SLOTS;
  if (slot_bytes) *slot_bytes = INFEROP_SPLITK_WS_BYTES + 4ll * INFEROP_SPLITK_WS_COUNTERS;
  return INFEROP_OK;
}

extern "C" int inferop_gemm_select(int64_t m, int64_t n, int64_t k, int32_t* config,
                                   int32_t* split_k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 128 != 0 || !config || !split_k) return INFEROP_ERR_ARGUMENT;
  const DeviceEntry* d = current_device();
  const GemmChoice ch = choose_gemm(m, n, k, d ? d->cus : 256);
  *config = ch.cfg;
  *split_k = ch.split;
  return INFEROP_OK;
}

extern "C" int inferop_diag_read_stream(const void* src, int64_t bytes, int32_t blocks,
                                        void* sink, void* stream) {
  if (!current_device()) return INFEROP_ERR_DEVICE;
  if (!src || !sink || bytes < 16 || bytes % 16 != 0 || blocks < 1 || blocks > (1 << 20))
    return INFEROP_ERR_ARGUMENT;
  return status_of_hip(
      inferop_hip_diag_read_stream(src, bytes, blocks, static_cast<uint32_t*>(sink), stream));
}

extern "C" int inferop_diag_stripe_read(const void* b, int64_t n, int64_t k, int32_t pattern,
                                        int32_t stripes, void* sink, void* stream) {
  if (!current_device()) return INFEROP_ERR_DEVICE;
  const int64_t g = k / 1024;
  if (!b || !sink || n < 16 || n % 16 != 0 || n / 16 > 65535 || k % 1024 != 0 ||
      (g != 2 && g != 7 && g != 8) || pattern < 0 || pattern > 4 || stripes < 0 ||
      stripes > n / 16)
    return INFEROP_ERR_ARGUMENT;
  return status_of_hip(inferop_hip_diag_stripe_read(b, n, k, pattern, stripes,
                                                    static_cast<uint32_t*>(sink), stream));
}

extern "C" int inferop_diag_mfma_loop(int32_t iters, int32_t blocks, int32_t promote, void* sink,
                                      void* stream) {
  if (!gemm_device()) return INFEROP_ERR_DEVICE;
  if (!sink || iters < 1 || blocks < 1 || blocks > (1 << 20)) return INFEROP_ERR_ARGUMENT;
  return status_of_hip(inferop_hip_diag_mfma_loop(iters, blocks, promote ? 1 : 0,
                                                  static_cast<uint32_t*>(sink), stream));
}

extern "C" int inferop_selftest_fp8_codec(uint64_t lo, uint64_t hi, uint64_t* counts,
                                          void* stream) {
  if (!current_device()) return INFEROP_ERR_DEVICE;
  return status_of_hip(inferop_hip_selftest_fp8_codec(lo, hi, counts, stream));
}
