"""Host-side checks that need no GPU: the library loads and exports every
symbol the headers declare, the drop-in C++ API links against a program built
from the reference's own ops.h, and argument guards behave like the
reference (nothing is launched without a device)."""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

import inferop_amd
from inferop_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include", "inferop")
REF_OPS = "/root/reference/include/inferop/ops.h"


def _c_declared_functions():
    text = open(os.path.join(INCLUDE, "inferop_c.h")).read()
    return sorted(set(re.findall(r"\b(inferop_[a-z0-9_]+)\s*\(", text)))


def _dynamic_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_library_loads():
    assert os.path.exists(_lib.LIB_PATH)
    inferop_amd.lib()


def test_exports_every_c_abi_symbol():
    declared = _c_declared_functions()
    assert len(declared) >= 12
    syms = _dynamic_symbols()
    missing = [d for d in declared if d not in syms]
    assert not missing, missing
    bound = {name for name, _, _ in _lib.C_API}
    assert set(declared) == bound


OPS_MANGLED = [
    "_ZN7inferop8has_cudaEv",
    "_ZN7inferop12device_countEv",
    "_ZN7inferop11device_nameEi",
    "_ZN7inferop17device_sm_versionEi",
    "_ZN7inferop25quant_fp8_per_token_groupEPvS0_PKvNS_5dtypeElliS0_",
    "_ZN7inferop27dequant_fp8_per_token_groupEPvNS_5dtypeEPKvS3_lliS0_",
    "_ZN7inferop19w8a8_block_fp8_gemmEPvPKvS2_S2_S2_llliiNS_5dtypeES0_",
    "_ZN7inferop12topk_softmaxEPiPvPKviiibS1_",
]


def test_exports_ops_h_mangled_symbols():
    syms = _dynamic_symbols()
    missing = [s for s in OPS_MANGLED if s not in syms]
    assert not missing, missing


DRIVER = r"""
#include <cstdio>
#include "inferop/ops.h"
int main() {
  using namespace inferop;
  std::printf("has=%d count=%d name=%s sm=%d\n", int(has_cuda()), device_count(),
              device_name(), device_sm_version());
  // guard paths only: no device pointers are dereferenced
  quant_fp8_per_token_group(nullptr, nullptr, nullptr, dtype::bf16, 4, 100, 128);
  w8a8_block_fp8_gemm(nullptr, nullptr, nullptr, nullptr, nullptr, 4, 8, 100);
  if (false) {
    topk_softmax(nullptr, nullptr, nullptr, 1, 8, 2);
    dequant_fp8_per_token_group(nullptr, dtype::bf16, nullptr, nullptr, 1, 128);
    w8a8_block_fp8_gemm(nullptr, nullptr, nullptr, nullptr, nullptr, 1, 1, 128, 128, 128,
                        dtype::fp16, nullptr);
  }
  return 0;
}
"""


def _build_driver(tmp_path, include_dir):
    src = tmp_path / "driver.cpp"
    src.write_text(DRIVER)
    exe = tmp_path / "driver"
    subprocess.run(["g++", "-std=c++17", "-O1", f"-I{include_dir}", str(src), "-o", str(exe),
                    f"-L{os.path.dirname(_lib.LIB_PATH)}", "-linferop",
                    f"-Wl,-rpath,{os.path.dirname(_lib.LIB_PATH)}"], check=True)
    return exe


def test_cpp_drop_in_links_and_guards(tmp_path):
    exe = _build_driver(tmp_path, os.path.join(ROOT, "include"))
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120,
                       env={**os.environ, "HIP_VISIBLE_DEVICES": os.environ.get("HIP_VISIBLE_DEVICES", "")})
    assert r.returncode == 0, r.stderr
    assert "unsupported shape (m=4 n=8 k=100 gs=128 bn=128)" in r.stderr


@pytest.mark.skipif(not os.path.exists(REF_OPS), reason="reference headers not present")
def test_program_built_against_reference_ops_h_links(tmp_path):
    # the same driver compiled against the REFERENCE's ops.h must resolve every
    # symbol from libinferop.so: the Itanium-mangled names are identical
    exe = _build_driver(tmp_path, "/root/reference/include")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr


def test_quant_guards_without_touching_memory():
    S = inferop_amd.Status
    q = inferop_amd.quant_fp8_per_token_group
    assert q(0, 0, 0, inferop_amd.dtype.bf16, 16, 100, 128) == S.ERR_SHAPE   # cols % gs
    assert q(0, 0, 0, inferop_amd.dtype.bf16, 0, 128, 128) == S.ERR_SHAPE
    assert q(0, 0, 0, inferop_amd.dtype.bf16, 4, 128, 0) == S.ERR_SHAPE
    assert q(0, 0, 0, inferop_amd.dtype.bf16, 4, -128, 128) == S.ERR_SHAPE
    assert q(0, 0, 0, inferop_amd.dtype.fp8_e4m3, 4, 128, 128) == S.ERR_DTYPE
    assert q(0, 0, 0, 7, 4, 128, 128) == S.ERR_DTYPE
    d = inferop_amd.dequant_fp8_per_token_group
    assert d(0, inferop_amd.dtype.fp32, 0, 0, 4, 130, 128) == S.ERR_SHAPE
    assert d(0, inferop_amd.dtype.fp8_e4m3, 0, 0, 4, 128, 128) == S.ERR_DTYPE
    w = inferop_amd.quant_fp8_weight_block
    assert w(0, 0, 0, inferop_amd.dtype.fp32, 128, 100) == S.ERR_SHAPE
    assert w(0, 0, 0, inferop_amd.dtype.fp32, 0, 128) == S.ERR_SHAPE
    assert w(0, 0, 0, inferop_amd.dtype.fp32, 128, 128, group_size=64) == S.ERR_SHAPE
    assert w(0, 0, 0, inferop_amd.dtype.fp32, 128, 128, block_n=256) == S.ERR_SHAPE
    assert w(0, 0, 0, inferop_amd.dtype.fp8_e4m3, 128, 128) == S.ERR_DTYPE
    assert w(16, 0, 8, inferop_amd.dtype.bf16, 128, 128) == S.ERR_ARGUMENT
    f = inferop_amd.silu_and_mul_quant_fp8
    assert f(0, 0, 0, inferop_amd.dtype.bf16, 4, 200) == S.ERR_SHAPE
    assert f(0, 0, 0, inferop_amd.dtype.bf16, 0, 256) == S.ERR_SHAPE
    assert f(0, 0, 0, inferop_amd.dtype.bf16, 4, 256, group_size=64) == S.ERR_SHAPE
    assert f(0, 0, 0, inferop_amd.dtype.fp8_e4m3, 4, 256) == S.ERR_DTYPE
    assert f(0, 0, 8, inferop_amd.dtype.bf16, 4, 256) == S.ERR_ARGUMENT
    t = inferop_amd.topk_softmax
    assert t(0, 0, 0, 4, 1025, 2) == S.ERR_SHAPE
    assert t(0, 0, 0, 4, 8, 9) == S.ERR_SHAPE
    assert t(0, 0, 0, 0, 8, 2) == S.ERR_SHAPE
    h = inferop_amd.fused_add_rmsnorm_quant_fp8
    assert h(0, 0, 0, 0, 0, inferop_amd.dtype.bf16, 4, 100) == S.ERR_SHAPE
    assert h(0, 0, 0, 0, 0, inferop_amd.dtype.fp8_e4m3, 4, 128) == S.ERR_DTYPE
    assert h(0, 0, 0, 0, 8, inferop_amd.dtype.bf16, 4, 128) == S.ERR_ARGUMENT


def test_gemm_guards_print_reference_diagnostic(capfd):
    S = inferop_amd.Status
    g = inferop_amd.w8a8_block_fp8_gemm
    assert g(0, 0, 0, 0, 0, 16, 512, 1000) == S.ERR_SHAPE
    assert g(0, 0, 0, 0, 0, 16, 512, 1024, group_size=64) == S.ERR_SHAPE
    assert g(0, 0, 0, 0, 0, 16, 512, 1024, block_n=64) == S.ERR_SHAPE
    assert g(0, 0, 0, 0, 0, 0, 512, 1024) == S.ERR_SHAPE
    err = capfd.readouterr().err
    assert err.count("[inferop] w8a8_block_fp8_gemm: unsupported shape") == 4
    assert "(m=16 n=512 k=1000 gs=128 bn=128); v0.1 requires gs=bn=128, k%128==0" in err
    # an unsupported output dtype is a silent no-op
    assert g(0, 0, 0, 0, 0, 16, 512, 1024, out_dt=inferop_amd.dtype.fp8_e4m3) == S.ERR_DTYPE
    assert capfd.readouterr().err == ""


def test_gemm_selection_covers_configs():
    # the gfx950 tile choice: decode tiles with split-K for M <= 64, prefill
    # tiles beyond; every choice names a valid kernel configuration
    n_cfg = inferop_amd.gemm_num_configs()
    names = [inferop_amd.gemm_config_name(i) for i in range(n_cfg)]
    assert len(set(names)) == n_cfg
    for m in (1, 16, 17, 64, 65, 77, 128, 1000, 4096, 8192):
        for n, k in ((7168, 2048), (4096, 7168), (2112, 7168), (4672, 7168), (32768, 512)):
            cfg, split = inferop_amd.gemm_select(m, n, k)
            assert 0 <= cfg < n_cfg
            assert 1 <= split <= k // 128
    # a long K over too few weight stripes to occupy every CU is split
    assert inferop_amd.gemm_select(1, 512, 8 * 7168)[1] > 1
    assert inferop_amd.gemm_select(1, 4096, 7168)[1] == 1
    # decode shapes: wide decode kernels for long K or few stripes, the
    # LDS-staged decode kernel for short K over many stripes, 128x32 tiles
    # with split-K when M > 32 leaves most CUs without a stripe
    def sel(m, n, k):
        cfg, split = inferop_amd.gemm_select(m, n, k)
        return names[cfg], split
    # M <= 8: 8-row activation tiles
    assert sel(1, 7168, 2048) == ("dw_m8_k4_w4a4", 1)
    assert sel(1, 4096, 7168) == ("dw_m8_k8_w4a4", 1)
    assert sel(8, 2112, 7168) == ("dw_m8_k8_w4a4", 1)
    assert sel(1, 7168, 7168) == ("dw_m8_k4_w4a4", 1)
    assert sel(16, 7168, 2048) == ("dw_m16_k4_w3a3", 1)
    assert sel(16, 4096, 7168) == ("dw_m16_k8_w3a3", 1)
    assert sel(16, 2112, 7168) == ("dw_m16_k8_w3a3", 1)
    assert sel(16, 7168, 7168) == ("dw_m16_k4_w3a3", 1)
    assert sel(16, 36864, 7168) == ("dw_m16_k8_w2a2", 1)
    assert sel(16, 7168, 18432) == ("dw_m16_k2_w8a8", 1)
    # 17 <= M <= 32: the stripe kernel below 32 scale groups (64x64 LDS tiles
    # beyond two stripes per CU), 64x32 wide tiles with K split from 32 up
    assert sel(32, 7168, 2048) == ("dw_m32_k4_w2a2", 1)
    assert sel(24, 24576, 1536) == ("pre_n64_m64_w4_s4", 1)
    assert sel(32, 4096, 7168) == ("dw_n64_m32_k4_w2a2", 4)
    assert sel(24, 7168, 18432) == ("dw_n64_m32_k4_w2a2", 2)
    assert sel(24, 36864, 7168) == ("dw_n64_m32_k4_w2a2", 1)
    # 33 <= M <= 64: a workgroup per 64 (or 32) weight rows, K split to fill
    # one round of CUs; two 32-row activation tiles only when N's 64-row
    # groups are a multiple of 8 (the tiles of a row group share an XCD)
    assert sel(64, 7168, 2048) == ("dw_n64_m32_k4_w2a2", 1)
    assert sel(64, 4096, 7168) == ("dw_n64_m32_k4_w2a2", 2)
    assert sel(64, 2112, 7168) == ("dw_n32_m64_k4_w2a2", 3)
    assert sel(64, 36864, 7168) == ("pre_n128_m64_w8_s4", 2)
    # a long K that one round of 64x32 tiles covers only unsplit: 128x64 tiles
    assert sel(48, 7168, 18432) == ("pre_n128_m64_w8_s4", 4)
    assert sel(128, 7168, 2048) == ("dw_n64_m64_k4_w2a2", 1)
    assert sel(128, 4096, 512) == ("dw_n64_m32_k4_w2a2", 1)
    assert sel(128, 7168, 18432) == ("per_n128_m128_w4", 4)
    # more 128x128 tiles than CUs at M <= 128: one round of 256x128 tiles
    assert sel(128, 36864, 7168) == ("pre_n256_m128_w8_s3", 1)
    assert sel(96, 36864, 7168) == ("pre_n256_m128_w8_s3", 1)
    assert sel(128, 40960, 4096)[0] != "pre_n256_m128_w8_s3"
    # M in (64, 128], fewer 128x128 tiles than CUs, 64-row groups a multiple
    # of 8: 64x64 wide decode tiles when they fill the CUs
    assert sel(100, 4096, 7168) == ("dw_n64_m64_k4_w2a2", 2)
    assert sel(96, 7168, 7168) == ("dw_n64_m64_k4_w2a2", 1)
    assert sel(128, 2048, 4096) == ("dw_n64_m32_k4_w2a2", 2)
    assert sel(128, 4096, 16384) == ("dw_n64_m64_k4_w2a2", 2)
    # ... 32-row activation tiles where they fill the CUs on their own or with
    # K split; a small weight whose row groups are not a multiple of 8 over
    # at most six of them; 64x64 LDS-staged tiles otherwise, at most 6 splits
    assert sel(72, 4608, 7168) == ("dw_n64_m32_k4_w2a2", 1)
    assert sel(96, 1536, 7168) == ("dw_n64_m32_k4_w2a2", 3)
    assert sel(96, 576, 7168) == ("dw_n64_m32_k4_w2a2", 7)
    assert sel(77, 4672, 7168)[0] == "pre_n64_m64_w4_s4"
    assert sel(128, 2112, 7168) == ("pre_n64_m64_w4_s4", 6)
    # beyond one round of two 64x64 tiles per CU: 128x128 tiles, or the
    # persistent ones with their tail split over a long K
    assert sel(96, 24576, 1536) == ("pre_n128_m128_w4_s2", 1)
    assert sel(96, 18432, 7168) == ("per_n128_m128_w4", 8)
    # 129 to 512 rows with fewer 128x128 tiles than CUs: wide decode tiles,
    # 64x64 LDS-staged tiles, persistent 128x128 tiles from 48 scale groups,
    # 128x128 tiles with the partials of a split within half the weight bytes
    assert sel(160, 1536, 7168) == ("dw_n64_m32_k4_w2a2", 2)
    assert sel(192, 4096, 7168) == ("dw_n64_m64_k4_w2a2", 1)
    assert sel(160, 4096, 8192) == ("dw_n64_m64_k4_w2a2", 1)
    assert sel(192, 576, 7168) == ("dw_n64_m32_k4_w2a2", 4)
    assert sel(448, 2048, 10240) == ("pre_n64_m64_w4_s4", 2)  # M x K > 4 MB
    assert sel(384, 576, 7168) == ("pre_n64_m64_w4_s4", 4)
    assert sel(192, 7168, 2048) == ("pre_n64_m64_w4_s4", 1)
    assert sel(160, 6144, 4096) == ("pre_n64_m64_w4_s4", 1)
    assert sel(384, 4096, 7168) == ("per_n128_m128_w4", 8)
    assert sel(448, 6144, 4096) == ("pre_n128_m128_w4_s2", 1)
    assert sel(224, 8192, 4096) == ("pre_n64_m64_w4_s4", 1)
    assert sel(320, 8192, 4096) == ("pre_n128_m128_w4_s2", 1)
    # up to 256 rows with many 128x128 tiles and a long K: persistent 256x256
    assert sel(160, 18432, 7168) == ("per_n256_m256_w8", 3)
    assert sel(160, 24576, 1536) == ("pre_n128_m128_w4_s2", 1)
    # fewer 256x256 tiles than CUs, at least as many 128x128 tiles, a long K:
    # persistent 256x256 tiles cut along K (configs[4] M=1000)
    assert sel(1000, 4672, 7168) == ("per_n256_m256_w8", 3)
    assert sel(1024, 7168, 2048) == ("pre_n128_m128_w4_s2", 1)
    # 256x256 prefill tiles run on the persistent kernel when K / 128 is even,
    # on the one-tile-per-workgroup kernel otherwise
    assert names[inferop_amd.gemm_select(4096, 7168, 16384)[0]] == "per_n256_m256_w8"
    assert names[inferop_amd.gemm_select(4096, 7168, 16384 + 128)[0]] == "pre_n256_m256_w8_s2"


def test_grouped_gemm_host_checks():
    # checked before any device work: shape and dtype errors, the m = 0
    # no-op, forced configurations without a grouped variant, and the tile
    # height chosen from the mean rows per expert
    S = inferop_amd.Status
    g = inferop_amd.w8a8_block_fp8_grouped_gemm
    assert g(0, 0, 0, 0, 0, 0, 16, 512, 1000, 8) == S.ERR_SHAPE
    assert g(0, 0, 0, 0, 0, 0, 16, 512, 1024, 0) == S.ERR_SHAPE
    assert g(0, 0, 0, 0, 0, 0, -1, 512, 1024, 8) == S.ERR_SHAPE
    assert g(0, 0, 0, 0, 0, 0, 16, 512, 1024, 8, group_size=64) == S.ERR_SHAPE
    assert g(0, 0, 0, 0, 0, 0, 16, 512, 1024, 8, out_dt=inferop_amd.dtype.fp8_e4m3) == S.ERR_DTYPE
    assert g(0, 0, 0, 0, 0, 0, 0, 512, 1024, 8) == S.OK
    names = [inferop_amd.gemm_config_name(i) for i in range(inferop_amd.gemm_num_configs())]
    gc = inferop_amd.w8a8_block_fp8_grouped_gemm_config
    for i, name in enumerate(names):
        if name not in ("pre_n128_m128_w4_s2", "pre_n128_m64_w8_s4", "pre_n128_m32_w8_s4",
                        "pre_n128_m16_w8_s4", "pre_n128_m64_w8_s3", "per_n256_m256_w8",
                        "per_n256_m128_w8", "per_n128_m128_w4", "dw_m16_k8_w3a3",
                        "dw_m16_k4_w3a3", "dw_m32_k4_w2a2", "dw_m64_k4_w2a2"):
            assert gc(0, 0, 0, 0, 0, 0, 16, 512, 1024, 8, inferop_amd.dtype.bf16, i) == \
                S.ERR_ARGUMENT, name
    gm = inferop_amd.w8a8_block_fp8_grouped_gemm_masked
    assert gm(0, 0, 0, 0, 0, 0, 8, 512, 1000, 8) == S.ERR_SHAPE
    assert gm(0, 0, 0, 0, 0, 0, -1, 512, 1024, 8) == S.ERR_SHAPE
    assert gm(0, 0, 0, 0, 0, 0, 1 << 20, 512, 1024, 1 << 12) == S.ERR_SHAPE  # rows past 2^31
    assert gm(0, 0, 0, 0, 0, 0, 0, 512, 1024, 8) == S.OK
    gmc = inferop_amd.w8a8_block_fp8_grouped_gemm_masked_config
    assert gmc(0, 0, 0, 0, 0, 0, 8, 512, 1024, 8, inferop_amd.dtype.bf16,
               names.index("pre_n256_m256_w8_s2")) == S.ERR_ARGUMENT
    # the persistent grouped kernels take an even K / 128
    assert gc(0, 0, 0, 0, 0, 0, 16, 512, 1152, 8, inferop_amd.dtype.bf16,
              names.index("per_n256_m256_w8")) == S.ERR_ARGUMENT
    # even K / 128: the persistent kernels; odd: the tiled ones
    sel = lambda m, e: names[inferop_amd.grouped_gemm_select(m, 4096, 7168, e)]
    # up to 8 rows per expert: the wide decode kernel over (stripe, expert tile)
    assert sel(64 * 8, 256) == "dw_m16_k4_w3a3"
    assert sel(8 * 32, 32) == "dw_m16_k4_w3a3"
    assert sel(9 * 32, 32) == "per_n128_m128_w4"
    assert sel(64 * 256, 256) == "per_n128_m128_w4"
    assert sel(128 * 256, 256) == "per_n256_m256_w8"
    sel = lambda m, e: names[inferop_amd.grouped_gemm_select(m, 4096, 7168 + 128, e)]
    assert sel(64 * 8, 256) == "dw_m16_k4_w3a3"
    assert sel(12 * 256, 256) == "pre_n128_m16_w8_s4"
    assert sel(20 * 256, 256) == "pre_n128_m32_w8_s4"
    assert sel(32 * 256, 256) == "pre_n128_m64_w8_s3"
    assert sel(64 * 256, 256) == "pre_n128_m128_w4_s2"
    assert sel(4096 * 8, 256) == "pre_n128_m128_w4_s2"


def test_persistent_config_rejects_odd_group_count():
    # checked before any device work: the persistent kernels need K / 128 even
    S = inferop_amd.Status
    g = inferop_amd.w8a8_block_fp8_gemm_config
    for i in range(inferop_amd.gemm_num_configs()):
        if inferop_amd.gemm_config_name(i).startswith("per_"):
            assert g(0, 0, 0, 0, 0, 256, 256, 384, inferop_amd.dtype.bf16, i, 1) == S.ERR_ARGUMENT


@pytest.mark.skipif(shutil.which("nm") is None, reason="binutils missing")
def test_no_cpu_fallback_symbols():
    # the product must not link the oracle
    syms = _dynamic_symbols()
    assert not any(s.startswith("orc_") or s.startswith("ref_") for s in syms)


SPLITK_WS_BYTES = 64 << 20  # INFEROP_SPLITK_WS_BYTES (inferop_amd/csrc/hip_launch.h)


def _tile_of(name):
    """(bn, bm) output tile of a split-capable configuration, from its name."""
    if name.startswith(("decl_", "dec_m16")):
        return 16, 16
    if name.startswith("dec_m"):
        return 16, int(name.split("_")[1][1:])
    if name.startswith("dw_m"):  # one 16-row weight stripe, bm activation rows
        return 16, int(name.split("_m")[1].split("_")[0])
    bn = int(name.split("_n")[1].split("_")[0])
    bm = int(name.split("_m")[1].split("_")[0])
    return bn, bm


def _workspace_bytes(cfg, split, m, n, k):
    f = inferop_amd.lib().inferop_hip_gemm_workspace_bytes
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
    return f(cfg, split, m, n, k)


def test_workspace_bytes_per_tile_of_every_split_configuration():
    # a tile's partial is stored as whole 16x16 blocks of 1 KB (the fixup's
    # layout): bn * ceil(bm / 16) * 16 * 4 bytes per tile and split, also for
    # the 8-row activation tiles, whose partial still fills 16-row blocks
    names = [inferop_amd.gemm_config_name(i) for i in range(inferop_amd.gemm_num_configs())]
    m, n, k, split = 40, 1000, 7168, 3
    for cfg, name in enumerate(names):
        if name.startswith("per_"):
            continue
        bn, bm = _tile_of(name)
        tiles = -(-n // bn) * -(-m // bm)
        want = split * tiles * bn * (-(-bm // 16) * 16) * 4
        assert _workspace_bytes(cfg, split, m, n, k) == want, name
        assert _workspace_bytes(cfg, 1, m, n, k) == 0, name
    m8 = names.index("dw_m8_k8_w4a4")
    assert _workspace_bytes(m8, 32, 1, 65536, 7168) == 32 * 4096 * 1024


def test_forced_split_of_8_row_tiles_beyond_workspace_is_rejected():
    # m=1, n=65536, split 32 on the 8-row wide decode tiles needs 128 MiB of
    # partials (4096 stripes x 1 KB x 32), twice a workspace slot
    S = inferop_amd.Status
    names = [inferop_amd.gemm_config_name(i) for i in range(inferop_amd.gemm_num_configs())]
    g = inferop_amd.w8a8_block_fp8_gemm_config
    for name in ("dw_m8_k8_w4a4", "dw_m8_k4_w4a4"):
        cfg = names.index(name)
        assert g(0, 0, 0, 0, 0, 1, 65536, 7168, inferop_amd.dtype.bf16, cfg, 32) == S.ERR_ARGUMENT
        # 16 splits need exactly the 64 MiB: not rejected for the workspace
        assert g(0, 0, 0, 0, 0, 1, 65536, 7168, inferop_amd.dtype.bf16, cfg, 16) != S.ERR_ARGUMENT


def test_automatic_split_fits_the_fixed_workspace():
    # the split-K workspace per stream has a fixed capacity and is never grown;
    # the automatic choice must stay within it at every shape, including a K
    # so long that the decode kernels would otherwise split it thousands of ways
    names = [inferop_amd.gemm_config_name(i) for i in range(inferop_amd.gemm_num_configs())]
    shapes = [(m, n, k) for m in (1, 8, 16, 33, 64, 65, 100, 128, 129, 300, 1000, 4096)
              for (n, k) in ((7168, 2048), (2112, 7168), (128, 65536), (36864, 7168),
                             (512, 1 << 20), (7168, 1 << 24), (64, 1 << 24))]
    for (m, n, k) in shapes:
        cfg, split = inferop_amd.gemm_select(m, n, k)
        if split == 1:
            continue
        bn, bm = _tile_of(names[cfg])
        bm = -(-bm // 16) * 16  # partials in whole 16-row blocks
        tiles = -(-n // bn) * -(-m // bm)
        if names[cfg].startswith("per_"):
            # persistent tiles: only the last, partial round's tiles are cut,
            # and their pieces fit one round of workgroups (256 CUs here)
            slots = 256 * (2 if bn * bm <= 128 * 128 else 1)
            tail = tiles % slots if tiles >= slots else tiles
            assert tail * split <= slots, (m, n, k, split)
            tiles = tail
        assert min(split, k // 128) * tiles * bn * bm * 4 <= SPLITK_WS_BYTES, (m, n, k, split)


def test_forced_split_beyond_workspace_is_rejected():
    # checked before any device work: a split whose partials exceed the fixed
    # workspace is an argument error, one that fits is not rejected for it
    S = inferop_amd.Status
    names = [inferop_amd.gemm_config_name(i) for i in range(inferop_amd.gemm_num_configs())]
    g = inferop_amd.w8a8_block_fp8_gemm_config
    cfg = names.index("pre_n128_m128_w4_s2")
    # 4096 x 4096 output = 1024 tiles of 64 KB: split 2 needs 128 MB
    assert g(0, 0, 0, 0, 0, 4096, 4096, 4096, inferop_amd.dtype.bf16, cfg, 2) == S.ERR_ARGUMENT
    # 256 x 256 output = 4 tiles: split 32 needs 8 MB (passes the check; without
    # a device the call then stops at the device check)
    assert g(0, 0, 0, 0, 0, 256, 256, 4096, inferop_amd.dtype.bf16, cfg, 32) != S.ERR_ARGUMENT


def test_masked_selection_checks_the_launch_grid():
    # the wide decode kernel's grid holds ceil(E * max_m / 16) + E rows of
    # workgroups (at most 65535): a small expected_m must not pick it when the
    # launch rows exceed that
    names = [inferop_amd.gemm_config_name(i) for i in range(inferop_amd.gemm_num_configs())]
    sel = lambda max_m, e, exp: names[inferop_amd.grouped_gemm_masked_select(max_m, 4096, 7168,
                                                                             e, exp)]
    assert sel(64, 32, 4) == "dw_m16_k4_w3a3"
    assert sel(4096, 256, 4) != "dw_m16_k4_w3a3"
    assert sel(4096, 256, 4).startswith("per_")
    assert sel(1024, 64, 8) == "dw_m16_k4_w3a3"  # 4096 + 64 rows of workgroups
