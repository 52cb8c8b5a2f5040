// TEST DRIVER (host code only, built with AddressSanitizer and
// UndefinedBehaviorSanitizer by `make -C tests/native sanitize`): runs the
// product's host layer (inferop_amd/csrc/ops.cpp: argument guards, gfx950 tile
// selection, C-ABI), the product's host headers (include/inferop/fp8.h,
// common.h, inferop_amd/csrc/quant_math.h) and the CPU oracle (oracle/oracle.c)
// over edge cases: ragged and extreme shapes, odd group sizes, special values.
// The HIP launch layer is replaced by the stubs below, which check the
// arguments the host layer passes and launch nothing.  Exit status 0 and no
// sanitizer report = pass.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <vector>

#include "hip_launch.h"
#include "inferop/common.h"
#include "inferop/fp8.h"
#include "inferop/inferop_c.h"
#include "quant_math.h"
#include "oracle.h"

namespace {
int g_fail = 0;
void check(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAIL: %s\n", what);
    ++g_fail;
  }
}
int32_t g_last_cfg = -1, g_last_split = -1;
constexpr int kStubConfigs = 36;
}  // namespace

// ---- stand-ins for the HIP launch layer (hip_launch.h) ----------------------
extern "C" {
int inferop_hip_device_count(void) { return 1; }
int inferop_hip_device_info(int ordinal, char* name, int name_len, int* arch, int* cu_count) {
  if (ordinal != 0) return 1;
  if (name && name_len > 0) std::snprintf(name, size_t(name_len), "%s", "stub gfx950");
  if (arch) *arch = 0x950;
  if (cu_count) *cu_count = 256;
  return 0;
}
int inferop_hip_current_device(int* ordinal) {
  *ordinal = 0;
  return 0;
}
int inferop_hip_quant_fp8_group(void*, float*, const void*, int32_t dt, int64_t rows, int64_t cols,
                                int32_t gs, void*) {
  check(dt >= 0 && dt <= 2 && rows > 0 && cols > 0 && gs > 0 && cols % gs == 0, "quant args");
  return 0;
}
int inferop_hip_dequant_fp8_group(void*, int32_t dt, const uint8_t*, const float*, int64_t rows,
                                  int64_t cols, int32_t gs, void*) {
  check(dt >= 0 && dt <= 2 && rows > 0 && cols > 0 && gs > 0 && cols % gs == 0, "dequant args");
  return 0;
}
int inferop_hip_weight_block_quant(uint8_t*, float*, const void*, int32_t dt, int64_t n, int64_t k,
                                   void*) {
  check(dt >= 0 && dt <= 2 && n > 0 && k > 0 && k % 128 == 0, "weight quant args");
  return 0;
}
int inferop_hip_silu_mul_quant(uint8_t*, float*, const void*, int32_t, int64_t t, int64_t d, void*) {
  check(t > 0 && d > 0 && d % 128 == 0, "silu args");
  return 0;
}
int inferop_hip_add_rmsnorm_quant(void*, uint8_t*, float*, const void*, const void*, int32_t,
                                  int64_t rows, int64_t cols, float, void*) {
  check(rows > 0 && cols > 0 && cols % 128 == 0, "rmsnorm args");
  return 0;
}
int inferop_hip_topk_softmax(int32_t*, float*, const float*, int tokens, int experts, int topk,
                             int, void*) {
  check(tokens > 0 && experts > 0 && experts <= 1024 && topk > 0 && topk <= experts, "topk args");
  return 0;
}
int inferop_hip_gemm_num_configs(void) { return kStubConfigs; }
int inferop_hip_gemm_config_info(int32_t cfg, inferop_gemm_cfg_info* info) {
  if (cfg < 0 || cfg >= kStubConfigs || !info) return 1;
  info->bn = 128;
  info->bm = 128;
  info->waves = 4;
  info->kind = (cfg >= 19 && cfg <= 21) ? 3 : (cfg >= 22 ? 4 : 2);
  info->name = "stub";
  info->grouped = 1;
  return 0;
}
int64_t inferop_hip_gemm_workspace_bytes(int32_t cfg, int32_t split, int64_t m, int64_t n,
                                         int64_t k) {
  if (cfg < 0 || cfg >= kStubConfigs || m <= 0 || n <= 0 || k < 128) return -1;
  if (split <= 1) return 0;
  // 128x128 fp32 partial tiles, as the tiled kernels need them
  const int64_t tiles = ((n + 127) / 128) * ((m + 127) / 128);
  if (tiles > INFEROP_SPLITK_WS_COUNTERS) return -1;
  int64_t s = split > k / 128 ? k / 128 : split;
  if (tiles > (int64_t(1) << 40) / (s * 65536)) return -1;
  return s * tiles * 65536;
}
// the workspace pool: INFEROP_SPLITK_WS_SLOTS streams take a slot each
void* g_slot_owner[INFEROP_SPLITK_WS_SLOTS];
int g_slots_used = 0;
int inferop_hip_splitk_reserve(void* stream) {
  for (int i = 0; i < g_slots_used; ++i)
    if (g_slot_owner[i] == stream) return 0;
  if (g_slots_used >= INFEROP_SPLITK_WS_SLOTS) return 2;  // hipErrorOutOfMemory
  g_slot_owner[g_slots_used++] = stream;
  return 0;
}
int inferop_hip_splitk_slots_used(void) { return g_slots_used; }
static int gemm_stub(const inferop_gemm_launch* l, int64_t m, int64_t n, int64_t k, int32_t dt) {
  check(l && l->cfg >= 0 && l->cfg < kStubConfigs, "gemm config in range");
  check(l && l->split_k >= 1 && l->split_k <= k / 128, "gemm split in range");
  check(m > 0 && n > 0 && k > 0 && k % 128 == 0 && dt >= 0 && dt <= 2, "gemm shape");
  g_last_cfg = l ? l->cfg : -1;
  g_last_split = l ? l->split_k : -1;
  return 0;
}
int inferop_hip_gemm_w8a8_block(void*, const uint8_t*, const float*, const uint8_t*, const float*,
                                int64_t m, int64_t n, int64_t k, int32_t dt,
                                const inferop_gemm_launch* l, void*) {
  return gemm_stub(l, m, n, k, dt);
}
int inferop_hip_gemm_w8a8_block_noalloc(void*, const uint8_t*, const float*, const uint8_t*,
                                        const float*, int64_t m, int64_t n, int64_t k, int32_t dt,
                                        const inferop_gemm_launch* l, void*) {
  return gemm_stub(l, m, n, k, dt);
}
int g_fused_launches = 0;
int inferop_hip_quant_gemm_decode(void*, uint8_t*, float*, const void*, int32_t dt, const uint8_t*,
                                  const float*, int64_t m, int64_t n, int64_t k, int32_t out_dt,
                                  int32_t waves, void*) {
  check(dt >= 0 && dt <= 2 && out_dt >= 0 && out_dt <= 2, "fused dtypes");
  check(m >= 1 && m <= 8 && n > 0 && k % 128 == 0, "fused shape");
  check((waves == 4 || waves == 8) && (k / 128 + waves - 1) / waves <= 8, "fused waves");
  ++g_fused_launches;
  return 0;
}
int inferop_hip_gemm_w8a8_block_grouped(void*, const uint8_t*, const float*, const uint8_t*,
                                        const float*, const int32_t*, int64_t m, int64_t n,
                                        int64_t k, int64_t experts, int64_t max_m, int32_t,
                                        int32_t cfg, void*) {
  check(cfg >= 0 && cfg < kStubConfigs, "grouped config");
  check(m >= 0 && n > 0 && k % 128 == 0 && experts > 0 && max_m >= 0, "grouped shape");
  return 0;
}
int inferop_hip_diag_read_stream(const void*, int64_t bytes, int32_t blocks, uint32_t*, void*) {
  check(bytes >= 16 && bytes % 16 == 0 && blocks >= 1, "read stream args");
  return 0;
}
int inferop_hip_diag_stripe_read(const void*, int64_t n, int64_t k, int32_t pattern,
                                 int32_t stripes, uint32_t*, void*) {
  check(n >= 16 && n % 16 == 0 && (k == 2048 || k == 7168 || k == 8192) && pattern >= 0 &&
            pattern <= 4 && stripes >= 0 && stripes <= n / 16,
        "stripe read args");
  return 0;
}
int inferop_hip_diag_mfma_loop(int32_t iters, int32_t blocks, int32_t, uint32_t*, void*) {
  check(iters >= 1 && blocks >= 1, "mfma loop args");
  return 0;
}
int inferop_hip_selftest_fp8_codec(uint64_t lo, uint64_t hi, uint64_t*, void*) {
  check(lo <= hi && hi <= (uint64_t(1) << 32), "selftest range");
  return 0;
}
}  // extern "C"

namespace {

float f_of(uint32_t w) {
  float f;
  std::memcpy(&f, &w, 4);
  return f;
}

void host_layer() {
  // every shape the selection may meet, extremes included: the chosen
  // configuration and split must be in range (checked by the stub)
  const int64_t ms[] = {1, 2, 15, 16, 17, 31, 32, 33, 48, 63, 64, 65, 77, 96, 127, 128, 129,
                        255, 256, 300, 511, 512, 1000, 1024, 2048, 4096, 8192, 65536, 1 << 20};
  const int64_t ns[] = {1, 7, 16, 100, 128, 256, 2112, 4096, 4672, 7168, 32768, 36864, 1 << 20};
  const int64_t ks[] = {128, 256, 512, 1024, 1536, 2048, 7168, 16384, 18432, 1 << 20,
                        int64_t(1) << 24};
  int launches = 0;
  for (int64_t m : ms)
    for (int64_t n : ns)
      for (int64_t k : ks) {
        if (m * n > (int64_t(1) << 34)) continue;
        int32_t cfg = -1, split = -1;
        check(inferop_gemm_select(m, n, k, &cfg, &split) == INFEROP_OK, "gemm_select ok");
        check(cfg >= 0 && cfg < kStubConfigs && split >= 1, "gemm_select range");
        int8_t dummy[16] = {};
        g_last_cfg = -1;
        check(inferop_w8a8_block_fp8_gemm(dummy, dummy, dummy, dummy, dummy, m, n, k, 128, 128, 2,
                                          nullptr) == INFEROP_OK,
              "gemm launch");
        check(g_last_cfg == cfg && g_last_split == split, "gemm launches the selected config");
        check(inferop_w8a8_block_fp8_gemm_noalloc(dummy, dummy, dummy, dummy, dummy, m, n, k, 128,
                                                  128, 1, nullptr) == INFEROP_OK,
              "noalloc launch");
        ++launches;
        int32_t g = -1;
        check(inferop_grouped_gemm_select(m, n, k, 32, &g) == INFEROP_OK, "grouped select");
        check(inferop_grouped_gemm_masked_select(m, n, k, 256, 4, &g) == INFEROP_OK ||
                  m * 256 > 0x7FFFFFFF,
              "masked select");
      }
  check(launches > 1000, "selection sweep ran");
  // the quantizer fused with the GEMM: one launch exactly where the plan says
  for (int64_t m : ms)
    for (int64_t n : ns)
      for (int64_t k : ks) {
        if (m * n > (int64_t(1) << 34) || m * k > (int64_t(1) << 34)) continue;
        alignas(16) int8_t buf[64] = {};
        const int before = g_fused_launches;
        check(inferop_quant_w8a8_block_fp8_gemm(buf, buf, buf, buf, 2, buf, buf, m, n, k, 128, 128,
                                                2, nullptr) == INFEROP_OK,
              "fused call");
        check((g_fused_launches - before == 1) ==
                  (inferop_quant_w8a8_block_fp8_gemm_launches(m, n, k) == 1),
              "fused launch count");
      }
  // rejected shapes and dtypes, including values that would overflow a product
  int8_t d[16] = {};
  check(inferop_w8a8_block_fp8_gemm(d, d, d, d, d, 4, 8, 100, 128, 128, 2, nullptr) ==
            INFEROP_ERR_SHAPE,
        "gemm k % 128");
  check(inferop_w8a8_block_fp8_gemm(d, d, d, d, d, -1, 8, 128, 128, 128, 2, nullptr) ==
            INFEROP_ERR_SHAPE,
        "gemm m < 0");
  check(inferop_w8a8_block_fp8_gemm(d, d, d, d, d, 4, 8, 128, 64, 128, 2, nullptr) ==
            INFEROP_ERR_SHAPE,
        "gemm group size");
  check(inferop_w8a8_block_fp8_gemm(d, d, d, d, d, 4, 8, 128, 128, 128, 3, nullptr) ==
            INFEROP_ERR_DTYPE,
        "gemm fp8 output");
  check(inferop_quant_fp8_per_token_group(d, d, d, 2, std::numeric_limits<int64_t>::max(), 128,
                                          128, nullptr) == INFEROP_OK,
        "quant huge rows reach the launch layer");
  check(inferop_quant_fp8_per_token_group(d, d, d, 2, 4, 130, 128, nullptr) == INFEROP_ERR_SHAPE,
        "quant cols % gs");
  check(inferop_quant_fp8_per_token_group(d, d, d, 2, 4, 128, 0, nullptr) == INFEROP_ERR_SHAPE,
        "quant gs 0");
  check(inferop_dequant_fp8_per_token_group(d, 7, d, d, 4, 128, 128, nullptr) == INFEROP_ERR_DTYPE,
        "dequant dtype");
  check(inferop_topk_softmax(nullptr, nullptr, nullptr, 4, 1025, 2, 1, nullptr) ==
            INFEROP_ERR_SHAPE,
        "topk experts");
  check(inferop_w8a8_block_fp8_grouped_gemm_masked(d, d, d, d, d, nullptr, int64_t(1) << 40, 128,
                                                   128, int64_t(1) << 30, 1, 128, 128, 2,
                                                   nullptr) == INFEROP_ERR_SHAPE,
        "masked rows overflow");
  check(inferop_w8a8_block_fp8_gemm_config(d, d, d, d, d, 4096, 4096, 4096, 2, 8, 64, nullptr) ==
            INFEROP_ERR_ARGUMENT,
        "forced split beyond the workspace");
  // workspace slots: once every slot belongs to a stream, a further stream's
  // automatic choice runs unsplit and a forced split on it is rejected
  {
    int32_t cfg = -1, split = -1;
    check(inferop_gemm_select(64, 2112, 7168, &cfg, &split) == INFEROP_OK && split > 1,
          "a split shape");
    char streams[INFEROP_SPLITK_WS_SLOTS + 1];
    for (int i = 0; i <= INFEROP_SPLITK_WS_SLOTS; ++i) {
      g_last_split = -1;
      check(inferop_w8a8_block_fp8_gemm(d, d, d, d, d, 64, 2112, 7168, 128, 128, 2,
                                        &streams[i]) == INFEROP_OK,
            "gemm on a new stream");
      const bool has_slot = i < INFEROP_SPLITK_WS_SLOTS - 1;  // the null stream holds one
      check(g_last_cfg == cfg && g_last_split == (has_slot ? split : 1), "split only with a slot");
    }
    int32_t used = -1, total = -1;
    int64_t bytes = -1;
    check(inferop_splitk_workspace_info(&used, &total, &bytes) == INFEROP_OK &&
              used == INFEROP_SPLITK_WS_SLOTS && total == INFEROP_SPLITK_WS_SLOTS &&
              bytes == INFEROP_SPLITK_WS_BYTES + 4 * INFEROP_SPLITK_WS_COUNTERS,
          "workspace info");
    check(inferop_w8a8_block_fp8_gemm_config(d, d, d, d, d, 64, 2112, 7168, 2, cfg, 2,
                                             &streams[INFEROP_SPLITK_WS_SLOTS]) ==
              INFEROP_ERR_ARGUMENT,
          "forced split without a slot");
    check(inferop_w8a8_block_fp8_gemm_config(d, d, d, d, d, 64, 2112, 7168, 2, cfg, 2, nullptr) ==
              INFEROP_OK,
          "forced split with a slot");
  }
  check(inferop_diag_read_stream(d, 8, 1, d, nullptr) == INFEROP_ERR_ARGUMENT, "read 8 bytes");
  check(inferop_diag_stripe_read(d, 4096, 3072, 0, 0, d, nullptr) == INFEROP_ERR_ARGUMENT,
        "stripe read k");
  check(inferop_diag_stripe_read(d, 100, 2048, 0, 0, d, nullptr) == INFEROP_ERR_ARGUMENT,
        "stripe read n");
  check(inferop_diag_stripe_read(d, 4096, 7168, 5, 0, d, nullptr) == INFEROP_ERR_ARGUMENT,
        "stripe read pattern");
  check(inferop_diag_stripe_read(d, 4096, 7168, 3, 16, d, nullptr) == INFEROP_OK,
        "stripe read resident");
  check(std::strcmp(inferop_status_string(99), "unknown status") == 0, "status text");
}

void host_headers() {
  // product conversions against the oracle on a strided sweep of fp32 bits
  for (uint64_t i = 0; i < (uint64_t(1) << 32); i += 65521) {
    const float f = f_of(uint32_t(i));
    check(inferop::fp8::float_to_e4m3_rn_sat(f) == orc_float_to_e4m3(f), "e4m3 encode");
    check(inferop::host_convert::float_to_bf16_rn(f) == orc_float_to_bf16(f), "bf16 encode");
    check(inferop::host_convert::float_to_half_rn(f) == orc_float_to_half(f), "fp16 encode");
  }
  for (int b = 0; b < 256; ++b) {
    const float x = inferop::fp8::e4m3_to_float(uint8_t(b)), y = orc_e4m3_to_float(uint8_t(b));
    check((std::isnan(x) && std::isnan(y)) || x == y, "e4m3 decode");
  }
  const float s = 3.0f * inferop_qmath::kInv448;
  check(inferop_qmath::div_by_recip(1.0f, s, 1.0f / s) == 1.0f / s, "quotient");
}

void oracle_edges() {
  const float inf = std::numeric_limits<float>::infinity();
  const float nan = std::numeric_limits<float>::quiet_NaN();
  for (int gs : {40, 48, 64, 128}) {
    const int64_t rows = 3, cols = 6 * gs;
    std::vector<float> x(size_t(rows * cols));
    for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(float(i)) * float(i % 7);
    x[1] = nan;
    x[2] = inf;
    x[size_t(gs)] = -inf;
    for (int i = 0; i < gs; ++i) x[size_t(2 * gs + i)] = 0.0f;  // a zero group
    x[size_t(3 * gs)] = 1e-42f;                                // denormal
    std::vector<uint8_t> q(x.size());
    std::vector<float> sc(size_t(rows * cols / gs)), back(x.size());
    orc_quant_fp8_per_token_group(q.data(), sc.data(), x.data(), rows, cols, gs);
    orc_dequant_fp8_per_token_group(back.data(), q.data(), sc.data(), rows, cols, gs);
  }
  // ragged GEMM: N not a multiple of 128, M = 1, rows subset, all threads
  const int64_t m = 5, n = 300, k = 256;
  std::vector<uint8_t> aq(size_t(m * k)), bq(size_t(n * k));
  for (size_t i = 0; i < aq.size(); ++i) aq[i] = uint8_t(i * 37);
  for (size_t i = 0; i < bq.size(); ++i) bq[i] = uint8_t(i * 91);
  std::vector<float> as(size_t(m * k / 128), 0.5f), bs(size_t(((n + 127) / 128) * (k / 128)), 2.f);
  std::vector<float> c(size_t(m * n)), cr(size_t(2 * n));
  orc_w8a8_block_fp8_gemm(c.data(), aq.data(), as.data(), bq.data(), bs.data(), m, n, k, 128, 128,
                          3);
  const int64_t rows[2] = {0, m - 1};
  orc_w8a8_block_fp8_gemm_rows(cr.data(), aq.data(), as.data(), bq.data(), bs.data(), m, n, k, 128,
                               128, rows, 2, 2);
  check(std::memcmp(cr.data(), c.data(), size_t(n) * 4) == 0, "gemm rows equal gemm");
  // weight blocks with a ragged last block row
  std::vector<float> w(size_t(n * k));
  for (size_t i = 0; i < w.size(); ++i) w[i] = std::cos(float(i)) * 0.02f;
  std::vector<uint8_t> wq(w.size());
  std::vector<float> wsc(size_t(((n + 127) / 128) * (k / 128)));
  orc_weight_block_quant(wq.data(), wsc.data(), w.data(), n, k, 128, 128);
  // fused producers
  std::vector<float> gu(size_t(2 * 3 * 128)), out(size_t(3 * 128)), res(size_t(3 * 128), 1.f);
  for (size_t i = 0; i < gu.size(); ++i) gu[i] = float(int(i) - 300) * 0.5f;
  orc_silu_and_mul(out.data(), gu.data(), 3, 128);
  std::vector<float> wt(128, 1.f);
  orc_rmsnorm(out.data(), gu.data(), wt.data(), 3, 128, 1e-6f);
  orc_fused_add_rmsnorm(res.data(), out.data(), gu.data(), wt.data(), 3, 128, 1e-6f);
  // routing: ties, one expert, top-k = all experts, 1024 experts
  for (int e : {1, 8, 257, 1024}) {
    std::vector<float> lg(size_t(2 * e), 0.25f);
    lg[0] = 3.0f;
    std::vector<int32_t> ids(size_t(2 * e));
    std::vector<float> wts(size_t(2 * e));
    orc_topk_softmax(ids.data(), wts.data(), lg.data(), 2, e, e, 1);
    orc_topk_softmax(ids.data(), wts.data(), lg.data(), 2, e, 1, 0);
  }
  // codec sweeps over small ranges, both ends of the bit space
  check(orc_sweep_encode_vs_grid(0, 1 << 16) == 0, "encode vs grid low");
  check(orc_sweep_encode_vs_grid(0xFFFF0000ull, 0x100000000ull) == 0, "encode vs grid high");
  std::vector<uint8_t> e8(4096);
  std::vector<uint16_t> e16(4096);
  orc_encode_range(0x7F7FF000ull, 0x7F800000ull + 0, e8.data());
  orc_bf16_range(0xFFFFF000ull, 0x100000000ull, e16.data());
  orc_half_range(0x477FF000ull, 0x47800000ull, e16.data());
  (void)orc_encode_checksum(0, 1 << 12);
  check(orc_grid_encode(448.0f) == 0x7E && orc_grid_encode(-nan) >= 0x7F, "grid encode");
}

}  // namespace

int main() {
  host_layer();
  host_headers();
  oracle_edges();
  if (g_fail) {
    std::fprintf(stderr, "%d check(s) failed\n", g_fail);
    return 1;
  }
  std::printf("sanitize_check: all checks passed\n");
  return 0;
}
