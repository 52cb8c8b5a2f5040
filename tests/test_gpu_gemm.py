"""GPU blockwise-FP8 GEMM parity with the oracle (reference.cpp:93-110, fp64
accumulation) on all five BASELINE.json configs, to the stated tolerance
max|err| <= 1e-2 * rms(C_ref) + 1 bf16 ulp."""
import os

import numpy as np
import pytest
import torch

import datagen
import inferop_amd
import oracle
from gpu_util import (anchor_ref_rows, assert_gemm_close, assert_gemm_close_dev, bf16_dev, device,
                      gemm_ref_f64, out_to_f32, to_dev, to_np)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DT = inferop_amd.dtype
TORCH_OUT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _gemm(aq, as_, bq, bs, m, n, k, out="bf16", config=None, split=1):
    c = torch.full((m, n), float("nan"), dtype=TORCH_OUT[out], device="cuda:0")
    if config is None:
        st = inferop_amd.w8a8_block_fp8_gemm(c, aq, as_, bq, bs, m, n, k, 128, 128,
                                             getattr(DT, out))
    else:
        st = inferop_amd.w8a8_block_fp8_gemm_config(c, aq, as_, bq, bs, m, n, k,
                                                    getattr(DT, out), config, split)
    assert st == 0
    return c


def _host_case(m, n, k, seed, dist="normal"):
    a_bits, a_f32, bq, bs = datagen.gemm_case(m, n, k, seed, dist)
    aq, as_ = oracle.quant(a_f32)
    return a_bits, aq, as_, bq, bs


@pytest.mark.gpu
def test_config0_golden_end_to_end():
    # BASELINE config 0, expected output written by the reference's own code:
    # GPU quantizer on the bf16 activations, then the GPU GEMM
    device()
    g = np.load(os.path.join(GOLDEN, "config0.npz"))
    m, k = g["a_q"].shape
    n = g["b_q"].shape[0]
    a = bf16_dev(g["a_bits"])
    q, s = inferop_amd.quantize(a)
    assert np.array_equal(to_np(q), g["a_q"])
    assert np.array_equal(to_np(s).view(np.uint32), g["a_s"].view(np.uint32))
    c = _gemm(q, s, to_dev(g["b_q"]), to_dev(g["b_s"]), m, n, k)
    assert_gemm_close(out_to_f32(c), g["c_ref"], "config0")


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 16, 64])
@pytest.mark.parametrize("nk", [(7168, 2048), (4096, 7168), (2112, 7168)])
def test_config1_decode_full_parity(m, nk):
    device()
    n, k = nk
    print(f"config1 m={m} n={n} k={k}", flush=True)
    a_bits, aq, as_, bq, bs = _host_case(m, n, k, seed=100 + m)
    # the decode step as the caller runs it: GPU quantizer (every byte and
    # scale equal to the oracle's), then the GEMM on its outputs
    q, s = inferop_amd.quantize(bf16_dev(a_bits))
    assert np.array_equal(to_np(q), aq)
    assert np.array_equal(to_np(s).view(np.uint32), as_.view(np.uint32))
    c = _gemm(q, s, to_dev(bq), to_dev(bs), m, n, k)
    assert_gemm_close(out_to_f32(c), oracle.gemm(aq, as_, bq, bs), f"config1 {m}x{n}x{k}")


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k,out,rtol,atol", [
    (256, 256, 512, "fp32", 2e-3, 2e-2),
    (256, 256, 512, "bf16", 1e-2, 3e-2),
    (100, 180, 256, "fp32", 2e-3, 2e-2),
    (4096, 4096, 4096, "bf16", 1e-2, 3e-2),
])
def test_reference_gpu_cross_check(m, n, k, out, rtol, atol):
    """The reference's own GPU cross-check (tests/test_gemm.cpp:62-96) on its four
    cases: A and W from N(0, 1) in fp32, A quantized per token group
    (reference.cpp:65-80), W per 128x128 block with the reciprocal
    (test_gemm.cpp:28-45), and every element within atol + rtol * |want| of the
    CPU reference (test_util.h:44-63) with the reference's tolerances.  The
    reference draws from one mt19937 stream; these are seeded numpy draws of the
    same distributions.  The 4096^3 case compares every element with the
    float64 GPU reference, itself checked against the oracle on 64 rows."""
    device()
    print(f"reference cross-check {m}x{n}x{k} {out}", flush=True)
    g = datagen.rng(900 + m + k, 3)
    a = g.standard_normal((m, k), dtype=np.float32)
    w = g.standard_normal((n, k), dtype=np.float32)
    aq, as_ = oracle.quant(a)
    bq, bs = oracle.weight_block_quant(w)
    # the GPU quantizers produce the same bytes and scales
    q, s = inferop_amd.quantize(to_dev(a))
    assert np.array_equal(to_np(q), aq)
    assert np.array_equal(to_np(s).view(np.uint32), as_.view(np.uint32))
    cd = _gemm(q, s, to_dev(bq), to_dev(bs), m, n, k, out=out)
    if m <= 256:
        c = out_to_f32(cd)
        want = oracle.gemm(aq, as_, bq, bs).astype(np.float64)
        diff = np.abs(c.astype(np.float64) - want)
        tol = atol + rtol * np.abs(want)
    else:
        rows = np.unique(np.concatenate([[0, m - 1], g.integers(0, m, 62)]))
        ref = gemm_ref_f64(q, s, to_dev(bq), to_dev(bs))
        anchor_ref_rows(ref, oracle.gemm_rows(aq, as_, bq, bs, rows), rows, "4096^3")
        assert bool(torch.isfinite(cd).all())
        diff = (cd.double() - ref).abs()
        tol = atol + rtol * ref.abs()
    bad = diff > tol
    nbad, total = int(bad.sum()), int(np.prod(bad.shape))
    assert nbad == 0, f"{nbad}/{total} mismatch, worst excess {float((diff - tol).max()):.4g}"


@pytest.mark.gpu
@pytest.mark.parametrize("m", [77, 1000])
def test_config4_ragged_stress(m):
    device()
    n, k = 4608 + 64, 7168
    print(f"config4 m={m}", flush=True)
    a_bits, a_f32, bq, bs = datagen.gemm_case(m, n, k, seed=400 + m, dist="stress")
    # quantize on the GPU; bytes must equal the oracle's
    q, s = inferop_amd.quantize(bf16_dev(a_bits))
    aq, as_ = oracle.quant(a_f32)
    assert np.array_equal(to_np(q), aq)
    assert np.array_equal(to_np(s).view(np.uint32), as_.view(np.uint32))
    bqd, bsd = to_dev(bq), to_dev(bs)
    c = _gemm(q, s, bqd, bsd, m, n, k)
    rows = np.arange(m) if m <= 128 else np.unique(np.concatenate(
        [[0, m - 1, m - 2], np.random.default_rng(m).integers(0, m, 29)]))
    want = oracle.gemm_rows(aq, as_, bq, bs, rows)
    assert_gemm_close(out_to_f32(c)[rows], want, f"config4 m={m}")
    # every element, against the float64 GPU reference anchored to the oracle rows
    ref = gemm_ref_f64(q, s, bqd, bsd)
    anchor_ref_rows(ref, want, rows, f"config4 m={m}")
    assert_gemm_close_dev(c, ref, f"config4 m={m} all elements")


def _device_case(m, n, k, seed):
    """Large shapes: inputs generated on the GPU; A quantized by the GPU
    quantizer; weights block-quantized with torch (input preparation only --
    the oracle receives the very same bytes)."""
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    a = torch.randn((m, k), generator=g, device="cuda:0").to(torch.bfloat16)
    w = torch.randn((n, k), generator=g, device="cuda:0") * 0.02
    nb = (n + 127) // 128
    wp = torch.zeros((nb * 128, k), device="cuda:0")
    wp[:n] = w
    blk = wp.view(nb, 128, k // 128, 128).abs().amax(dim=(1, 3))
    inv448 = torch.tensor(1.0 / 448.0, dtype=torch.float32, device="cuda:0")
    bs = torch.where(blk == 0, torch.ones_like(blk), blk * inv448)
    inv = (1.0 / bs).repeat_interleave(128, 0).repeat_interleave(128, 1)[:n]
    bq = (w * inv).to(torch.float8_e4m3fn).view(torch.uint8)
    aq, as_ = inferop_amd.quantize(a)
    return a, aq, as_, bq.contiguous(), bs.contiguous()


def _check_full(a, aq, as_, bq, bs, outs, rows, what):
    """Every element of every output in `outs` against the float64 GPU
    reference; the reference is first checked against the oracle
    (reference.cpp:93-110) on the sampled rows.  The GPU quantizer's bytes
    and scales are compared with the oracle's quantizer (reference.cpp:65-80)
    over the whole activation tensor, every byte and every scale (the
    reference's own test compares every byte, tests/test_quant.cpp:62-63)."""
    qr, sr = oracle.quant(datagen.bf16_bits_to_f32(to_np(a)))
    q_all, s_all = to_np(aq), to_np(as_)
    nq = int((q_all != qr).sum())
    ns = int((s_all.view(np.uint32) != sr.view(np.uint32)).sum())
    assert nq == 0 and ns == 0, f"{what}: quantizer differs in {nq} bytes, {ns} scales"
    del qr, sr, q_all, s_all
    aq_h, as_h = to_np(aq[rows]), to_np(as_[rows])
    want = oracle.gemm_rows(aq_h, as_h, to_np(bq), to_np(bs), np.arange(len(rows)))
    ref = gemm_ref_f64(aq, as_, bq, bs)
    anchor_ref_rows(ref, want, rows, what)
    for name, c in outs.items():
        assert_gemm_close(out_to_f32(c[rows]), want, f"{what} {name} sampled rows")
        assert_gemm_close_dev(c, ref, f"{what} {name} all elements")


@pytest.mark.gpu
@pytest.mark.parametrize("nk", [(24576, 1536), (32768, 512), (7168, 16384), (4608, 7168)])
def test_config2_prefill_all_elements(nk):
    device()
    m = 4096
    n, k = nk
    print(f"config2 n={n} k={k}", flush=True)
    a, aq, as_, bq, bs = _device_case(m, n, k, seed=200)
    c = _gemm(aq, as_, bq, bs, m, n, k)
    rows = np.unique(np.concatenate([[0, 1, 4095], np.random.default_rng(n).integers(0, m, 9)]))
    _check_full(a, aq, as_, bq, bs, {"bf16": c}, rows, f"config2 {n}x{k}")


@pytest.mark.gpu
@pytest.mark.parametrize("m", [128, 512, 1024, 2048, 8192])
@pytest.mark.parametrize("nk", [(7168, 18432), (36864, 7168), (7168, 2048), (4096, 512)])
def test_config3_m_sweep_all_elements(m, nk):
    device()
    n, k = nk
    print(f"config3 m={m} n={n} k={k}", flush=True)
    a, aq, as_, bq, bs = _device_case(m, n, k, seed=300 + m)
    rows = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(m + n).integers(0, m, 4)]))
    outs = {out: _gemm(aq, as_, bq, bs, m, n, k, out=out) for out in ("bf16", "fp16")}
    _check_full(a, aq, as_, bq, bs, outs, rows, f"config3 {m}x{n}x{k}")


# One shape per branch of the automatic tile choice between the decode and
# the prefill sizes (17-512 rows), each named with the configuration and K
# split the host picks for it (checked by the host tests); every element of
# the automatically launched product is compared.
SELECTION_SHAPES = [
    (24, 4096, 7168),     # 64x32 wide tiles, K in 4
    (24, 24576, 1536),    # 64x64 LDS-staged tiles beyond two stripes per CU
    (48, 7168, 18432),    # 128x64 LDS-staged tiles, K in 4
    (72, 4608, 7168),     # 64x32 wide tiles unsplit
    (96, 576, 7168),      # 64x32 wide tiles, row groups not a multiple of 8
    (96, 24576, 1536),    # 128x128 tiles
    (96, 18432, 7168),    # persistent 128x128 tiles, tail split
    (160, 1536, 7168),    # 64x32 wide tiles, K in 2
    (192, 4096, 7168),    # 64x64 wide tiles
    (150, 1000, 7168),    # ragged N and M on wide tiles
    (448, 2048, 10240),   # 64x64 LDS-staged tiles, K in 2 (M x K beyond L2)
    (384, 4096, 7168),    # persistent 128x128 tiles, tail split
    (448, 6144, 4096),    # 128x128 tiles unsplit
    (300, 2500, 5120),    # ragged, 64x64 wide tiles
    (300, 2600, 5120),    # ragged, 64x64 LDS-staged tiles, K in 2
    (160, 18432, 7168),   # persistent 256x256 tiles, tail split
]


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k", SELECTION_SHAPES)
def test_selected_kernels_mid_m_all_elements(m, n, k):
    device()
    cfg, split = inferop_amd.gemm_select(m, n, k)
    what = f"m={m} n={n} k={k} {inferop_amd.gemm_config_name(cfg)}:{split}"
    print(what, flush=True)
    a, aq, as_, bq, bs = _device_case(m, n, k, seed=400 + m)
    rows = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(m * n).integers(0, m, 4)]))
    outs = {out: _gemm(aq, as_, bq, bs, m, n, k, out=out) for out in ("bf16", "fp16")}
    _check_full(a, aq, as_, bq, bs, outs, rows, what)


N_CONFIGS = inferop_amd.gemm_num_configs()


@pytest.mark.gpu
@pytest.mark.parametrize("config", range(N_CONFIGS))
@pytest.mark.parametrize("split", [1, 3])
def test_every_kernel_config_ragged(config, split):
    device()
    m, n, k = 77, 300, 768
    _, aq, as_, bq, bs = _host_case(m, n, k, seed=7, dist="stress")
    want = oracle.gemm(aq, as_, bq, bs)
    for out in ("bf16", "fp32"):
        c = _gemm(to_dev(aq), to_dev(as_), to_dev(bq), to_dev(bs), m, n, k, out, config, split)
        assert_gemm_close(out_to_f32(c), want, f"cfg{config} split{split} {out}")


def _shifted(t, shift_bytes):
    """A copy of t whose data starts shift_bytes past a 256-byte boundary
    (returned with the buffer that holds it)."""
    nbytes = t.numel() * t.element_size()
    raw = torch.zeros(nbytes + 512, dtype=torch.uint8, device=t.device)
    view = raw[shift_bytes:shift_bytes + nbytes]
    view.copy_(t.contiguous().view(torch.uint8).reshape(-1))
    out = view.view(t.dtype).reshape(t.shape)
    assert out.data_ptr() % 16 == shift_bytes % 16
    return raw, out


@pytest.mark.gpu
@pytest.mark.parametrize("config", range(N_CONFIGS))
def test_every_config_with_4_byte_aligned_pointers(config):
    # The reference asks only 4-byte alignment of its pointers
    # (kernels/gemm/w8a8_block_fp8.cu:64,78); the kernels load 16 bytes per
    # lane.  With every operand and C 4, 8 or 12 bytes past a 16-byte
    # boundary each configuration gives the bits of the aligned call (C then
    # takes the element-wise stores).
    device()
    m, n, k = 77, 300, 768
    _, aq, as_, bq, bs = _host_case(m, n, k, seed=11, dist="stress")
    want = oracle.gemm(aq, as_, bq, bs)
    aq, as_, bq, bs = to_dev(aq), to_dev(as_), to_dev(bq), to_dev(bs)
    name = inferop_amd.gemm_config_name(config)
    for out in ("bf16", "fp32"):
        c0 = _gemm(aq, as_, bq, bs, m, n, k, out, config, 1)
        held, ops = [], []
        for t, sh in ((aq, 4), (as_, 4), (bq, 8), (bs, 12)):
            raw, v = _shifted(t, sh)
            held.append(raw)
            ops.append(v)
        rawc, c1 = _shifted(torch.full((m, n), float("nan"), dtype=TORCH_OUT[out],
                                       device="cuda:0"), 4)
        st = inferop_amd.w8a8_block_fp8_gemm_config(c1, *ops, m, n, k, getattr(DT, out),
                                                    config, 1)
        assert st == 0
        assert_gemm_close(out_to_f32(c1), want, f"{name} {out} shifted")
        assert torch.equal(c0, c1), f"{name} {out}: shifted pointers change the result"


def _cfg(name):
    return next(i for i in range(N_CONFIGS) if inferop_amd.gemm_config_name(i) == name)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["per_n256_m256_w8", "per_n256_m128_w8", "per_n128_m128_w4"])
def test_persistent_kernels_match_tiled_kernel(name):
    # The persistent kernels walk several tiles per workgroup and keep the
    # load pipeline running across tile boundaries; per output element they
    # add the scale groups in the same order as the one-tile-per-workgroup
    # kernel, so the outputs are identical, ragged edges included.  Shapes:
    # many rounds of ragged tiles, the shortest K (two groups: no steady-state
    # iteration), and fewer tiles than CUs.
    device()
    ref = _cfg("pre_n256_m256_w8_s2")
    for (m, n, k) in [(4000, 9000, 512), (1500, 33000, 256), (700, 4100, 1536)]:
        print(f"{name} {m}x{n}x{k}", flush=True)
        a, aq, as_, bq, bs = _device_case(m, n, k, seed=m + n)
        for out in ("bf16", "fp16", "fp32"):
            want = _gemm(aq, as_, bq, bs, m, n, k, out, ref, 1)
            got = _gemm(aq, as_, bq, bs, m, n, k, out, _cfg(name), 1)
            assert torch.equal(got, want), f"{name} {m}x{n}x{k} {out}"
        rows = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(m).integers(0, m, 4)]))
        _check_full(a, aq, as_, bq, bs, {"fp32": got}, rows, f"{name} {m}x{n}x{k}")


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["per_n256_m256_w8", "per_n256_m128_w8", "per_n128_m128_w4"])
def test_persistent_tail_split(name):
    # split_k > 1 on a persistent configuration cuts the tiles of the last,
    # partial round into K ranges whose fp32 partials a second kernel adds in
    # piece order: every element within tolerance of the float64 reference,
    # and bit-identical from run to run.  Shapes: a partial last round after
    # full ones (4096 x 9216: 16 x 36 tiles of 256), fewer tiles than
    # workgroups, ragged M and N, and a split that leaves one pair of groups
    # per piece.
    device()
    for (m, n, k, split) in [(4096, 9216, 1024, 4), (700, 4100, 1536, 3), (333, 1000, 512, 2),
                             (512, 4608, 7168, 8)]:
        print(f"{name} tail split {split} {m}x{n}x{k}", flush=True)
        a, aq, as_, bq, bs = _device_case(m, n, k, seed=m + n + split)
        outs = {}
        for out in ("bf16", "fp32"):
            c = _gemm(aq, as_, bq, bs, m, n, k, out, _cfg(name), split)
            again = _gemm(aq, as_, bq, bs, m, n, k, out, _cfg(name), split)
            assert torch.equal(c, again), f"{name} {m}x{n}x{k} {out}: not repeatable"
            outs[out] = c
        rows = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(m).integers(0, m, 4)]))
        _check_full(a, aq, as_, bq, bs, outs, rows, f"{name} tail {split} {m}x{n}x{k}")


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["dw_m64_k4_w2a2", "dw_m64_k2_w4a2", "dw_m32_k4_w2a2",
                                  "dw_m16_k2_w8a8", "dw_m16_k8_w3a3", "dw_m16_k4_w3a3",
                                  "dw_m16_k8_w2a2", "dw_n64_m64_k4_w2a2", "dw_n32_m64_k4_w2a2",
                                  "dw_n64_m32_k4_w2a2", "dw_n32_m16_k8_w3a3",
                                  "dw_n32_m32_k8_w2a2"])
def test_wide_decode_kernels(name):
    # one workgroup per 16-row weight stripe over all of K: ragged stripes,
    # several activation tiles (M past one tile), waves left without groups
    # (K/128 below the wave count), odd group counts, every output dtype; the
    # last two shapes give some configurations more scale groups per wave than
    # the scale preload holds (the kernel without it)
    device()
    cfg = _cfg(name)
    cases = [(1, 2112, 7168), (5, 300, 256), (17, 4096, 2048), (48, 1000, 1152), (64, 2112, 7168),
             (70, 520, 384), (3, 640, 18432), (40, 520, 9216)]
    for (m, n, k) in cases:
        print(f"{name} {m}x{n}x{k}", flush=True)
        _, aq, as_, bq, bs = _host_case(m, n, k, seed=m + n)
        want = oracle.gemm(aq, as_, bq, bs)
        args = [to_dev(v) for v in (aq, as_, bq, bs)]
        for out in ("bf16", "fp16", "fp32"):
            c = _gemm(*args, m, n, k, out, cfg, 1)
            assert_gemm_close(out_to_f32(c), want, f"{name} {m}x{n}x{k} {out}")
            assert torch.equal(_gemm(*args, m, n, k, out, cfg, 1), c)  # no atomics: repeatable


@pytest.mark.gpu
def test_output_dtypes_and_odd_n():
    device()
    for (m, n, k) in [(40, 130, 256), (5, 7, 128), (129, 1, 384)]:
        _, aq, as_, bq, bs = _host_case(m, n, k, seed=m + n)
        want = oracle.gemm(aq, as_, bq, bs)
        for out in ("bf16", "fp16", "fp32"):
            c = _gemm(to_dev(aq), to_dev(as_), to_dev(bq), to_dev(bs), m, n, k, out)
            assert_gemm_close(out_to_f32(c), want, f"{m}x{n}x{k} {out}")


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 16, 64])
def test_split_k_deterministic_and_repeatable(m):
    # the split-K partials cross workgroups (and XCDs) through device-coherent
    # stores; repeated runs must agree bit for bit with each other and, in
    # tolerance, with the oracle, for every split count
    device()
    n, k = 2112, 7168
    _, aq, as_, bq, bs = _host_case(m, n, k, seed=9)
    want = oracle.gemm(aq, as_, bq, bs)
    args = [to_dev(v) for v in (aq, as_, bq, bs)]
    cfg, _ = inferop_amd.gemm_select(m, n, k)
    for split in (2, 5, 14, 56):
        first = to_np(_gemm(*args, m, n, k, "fp32", cfg, split))
        assert_gemm_close(first, want, f"split {split}")
        for _ in range(5):
            assert np.array_equal(to_np(_gemm(*args, m, n, k, "fp32", cfg, split)), first)


@pytest.mark.gpu
def test_gemm_rejected_calls_leave_output_untouched(capfd):
    device()
    c = torch.full((4, 8), 5.0, dtype=torch.float32, device="cuda:0")
    z = torch.zeros(1024, dtype=torch.uint8, device="cuda:0")
    S = inferop_amd.Status
    assert inferop_amd.w8a8_block_fp8_gemm(c, z, z, z, z, 4, 8, 100, out_dt=DT.fp32) == S.ERR_SHAPE
    assert inferop_amd.w8a8_block_fp8_gemm(c, z, z, z, z, 4, 8, 128,
                                           out_dt=DT.fp8_e4m3) == S.ERR_DTYPE
    torch.cuda.synchronize()
    assert (c == 5.0).all()
    assert "unsupported shape (m=4 n=8 k=100" in capfd.readouterr().err
