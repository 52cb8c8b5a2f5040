"""GPU grouped blockwise-FP8 GEMM over MoE experts, contiguous layout (the
reference's roadmap item docs/ROADMAP.md:39; no counterpart in its ops.h).

Row r of the activations belongs to the expert e whose segment
[offsets[e], offsets[e+1]) holds it and is multiplied by that expert's
weights, so the oracle is the plain GEMM oracle (reference.cpp:93-110) run on
each expert's rows against its weights, at the GEMM's tolerance.  The grouped
kernels are the tiled GEMM kernels with the expert's weights, so with the same
configuration each expert's rows also equal the plain GEMM of that segment
bit for bit."""
import numpy as np
import pytest
import torch

import datagen
import inferop_amd
import oracle
from gpu_util import assert_gemm_close, device, out_to_f32, to_dev

DT = inferop_amd.dtype
TORCH_OUT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
N_CONFIGS = inferop_amd.gemm_num_configs()
GROUPED = ["pre_n128_m128_w4_s2", "pre_n128_m64_w8_s4", "pre_n128_m32_w8_s4", "pre_n128_m16_w8_s4",
           "pre_n128_m64_w8_s3", "per_n256_m256_w8", "per_n256_m128_w8", "per_n128_m128_w4",
           "dw_m16_k8_w3a3", "dw_m16_k4_w3a3", "dw_m32_k4_w2a2", "dw_m64_k4_w2a2"]


def _cfg(name):
    return next(i for i in range(N_CONFIGS) if inferop_amd.gemm_config_name(i) == name)


def _experts(sizes, n, k, seed, dist="normal"):
    """Activations for sum(sizes) rows (quantized by the oracle) and one
    block-quantized weight matrix per expert."""
    m = int(sum(sizes))
    a_bits, a_f32, _, _ = datagen.gemm_case(max(m, 1), 16, k, seed, dist)
    aq, as_ = oracle.quant(a_f32[:m]) if m else (np.zeros((0, k), np.uint8),
                                                 np.zeros((0, k // 128), np.float32))
    bqs, bss = [], []
    for e in range(len(sizes)):
        bq, bs = oracle.weight_block_quant(datagen.weights(n, k, seed * 131 + e, dist))
        bqs.append(bq)
        bss.append(bs)
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    return aq, as_, np.stack(bqs), np.stack(bss), offsets


def _grouped(aq, as_, bq, bs, offsets, m, n, k, out="bf16", config=None):
    c = torch.full((max(m, 1), n), float("nan"), dtype=TORCH_OUT[out], device="cuda:0")
    e = len(offsets) - 1
    if config is None:
        st = inferop_amd.w8a8_block_fp8_grouped_gemm(c, aq, as_, bq, bs, offsets, m, n, k, e,
                                                     out_dt=getattr(DT, out))
    else:
        st = inferop_amd.w8a8_block_fp8_grouped_gemm_config(c, aq, as_, bq, bs, offsets, m, n, k,
                                                            e, getattr(DT, out), config)
    assert st == 0
    return c


@pytest.mark.gpu
@pytest.mark.parametrize("name", GROUPED)
def test_grouped_matches_oracle_per_expert(name):
    # empty experts (first, middle, last), one-row experts, segments that end
    # inside a tile and cross several, ragged N, every output dtype
    device()
    sizes = [0, 1, 17, 130, 64, 0, 5, 83, 33, 0]
    n, k = 520, 768
    aq, as_, bq, bs, offsets = _experts(sizes, n, k, seed=11)
    m = int(offsets[-1])
    args = [to_dev(v) for v in (aq, as_, bq, bs, offsets)]
    for out in ("bf16", "fp16", "fp32"):
        print(f"{name} {out}", flush=True)
        c = out_to_f32(_grouped(*args, m, n, k, out, _cfg(name)))
        for e in range(len(sizes)):
            r0, r1 = int(offsets[e]), int(offsets[e + 1])
            if r1 == r0:
                continue
            want = oracle.gemm(aq[r0:r1], as_[r0:r1], bq[e], bs[e])
            assert_gemm_close(c[r0:r1], want, f"{name} {out} expert {e}")


@pytest.mark.gpu
@pytest.mark.parametrize("name", GROUPED)
def test_grouped_equals_plain_gemm_per_segment(name):
    # the grouped kernel is the tiled kernel on the expert's weights with the
    # tile rows counted from the segment start: bit-identical to the plain
    # GEMM of each segment with the same configuration
    device()
    sizes = [37, 0, 200, 1, 128, 129]
    n, k = 384, 1024
    aq, as_, bq, bs, offsets = _experts(sizes, n, k, seed=5, dist="stress")
    m = int(offsets[-1])
    cfg = _cfg(name)
    A, S, B, BS, O = (to_dev(v) for v in (aq, as_, bq, bs, offsets))
    for out in ("bf16", "fp32"):
        got = _grouped(A, S, B, BS, O, m, n, k, out, cfg)
        for e in range(len(sizes)):
            r0, r1 = int(offsets[e]), int(offsets[e + 1])
            if r1 == r0:
                continue
            c = torch.empty((r1 - r0, n), dtype=TORCH_OUT[out], device="cuda:0")
            assert inferop_amd.w8a8_block_fp8_gemm_config(
                c, A[r0:r1], S[r0:r1], B[e], BS[e], r1 - r0, n, k, getattr(DT, out), cfg, 1) == 0
            assert torch.equal(got[r0:r1], c), f"{name} {out} expert {e}"
        # repeatable
        assert torch.equal(_grouped(A, S, B, BS, O, m, n, k, out, cfg), got)


@pytest.mark.gpu
def test_grouped_moe_shapes_sampled():
    # DeepSeek-V3-like expert shape (n = 2048, k = 7168: an expert's up
    # projection) with the automatic configuration: decode-sized (a few rows
    # per expert) and prefill-sized (hundreds) routings, sampled rows per
    # expert
    device()
    n, k = 2048, 7168
    for sizes, seed in (([3, 0, 1, 8, 2, 0, 5, 1], 21), ([300, 17, 0, 513, 96, 260, 128, 44], 22)):
        aq, as_, bq, bs, offsets = _experts(sizes, n, k, seed)
        m = int(offsets[-1])
        print(f"experts={len(sizes)} m={m} cfg="
              f"{inferop_amd.gemm_config_name(inferop_amd.grouped_gemm_select(m, n, k, len(sizes)))}",
              flush=True)
        c = out_to_f32(_grouped(*[to_dev(v) for v in (aq, as_, bq, bs, offsets)], m, n, k))
        rng = np.random.default_rng(seed)
        for e in range(len(sizes)):
            r0, r1 = int(offsets[e]), int(offsets[e + 1])
            if r1 == r0:
                continue
            rows = np.unique(np.concatenate([[0, r1 - r0 - 1], rng.integers(0, r1 - r0, 3)]))
            want = oracle.gemm_rows(aq[r0:r1], as_[r0:r1], bq[e], bs[e], rows)
            assert_gemm_close(c[r0 + rows], want, f"expert {e}")


@pytest.mark.gpu
def test_grouped_offsets_out_of_range_stay_in_bounds():
    # offsets are device data the host cannot check: the kernel clamps them to
    # [0, m] (and each end to at least its start), so decreasing or
    # out-of-range values only ever address rows of A and C; rows claimed by
    # one expert alone come out right (rows 30..39 are claimed twice here)
    device()
    sizes = [40, 40, 40]
    n, k = 256, 512
    aq, as_, bq, bs, offsets = _experts(sizes, n, k, seed=3)
    m = 120
    bad = np.array([-50, 40, 30, 1000], dtype=np.int32)  # expert 1 empty, expert 2 = [30, 120)
    c = _grouped(*[to_dev(v) for v in (aq, as_, bq, bs, bad)], m, n, k, "fp32",
                 _cfg("pre_n128_m64_w8_s4"))
    got = out_to_f32(c)
    assert_gemm_close(got[0:30], oracle.gemm(aq[0:30], as_[0:30], bq[0], bs[0]), "expert 0")
    assert_gemm_close(got[40:120], oracle.gemm(aq[40:120], as_[40:120], bq[2], bs[2]), "expert 2")


@pytest.mark.gpu
def test_grouped_rejected_calls():
    device()
    S = inferop_amd.Status
    g = inferop_amd.w8a8_block_fp8_grouped_gemm
    # m = 0: nothing to do, nothing written
    c = torch.full((4, 128), 7.0, device="cuda:0")
    assert g(c, 0, 0, 0, 0, 0, 0, 128, 256, 4, out_dt=DT.fp32) == S.OK
    assert torch.all(c == 7.0)
    assert g(c, 0, 0, 0, 0, 0, 4, 128, 200, 4) == S.ERR_SHAPE
    assert g(c, 0, 0, 0, 0, 0, 4, 128, 256, 0) == S.ERR_SHAPE
    assert g(c, 0, 0, 0, 0, 0, 4, 128, 256, 4, out_dt=DT.fp8_e4m3) == S.ERR_DTYPE
    assert torch.all(c == 7.0)


def _masked_inputs(counts, max_m, aq, as_, offsets):
    """Scatter the contiguous layout's expert segments into the masked layout
    [E, max_m, ...] (rows past a count: arbitrary bytes, never read as data)."""
    e_n = len(counts)
    k = aq.shape[1]
    a3 = np.random.default_rng(7).integers(0, 0x7E, (e_n, max_m, k), dtype=np.uint8)
    s3 = np.full((e_n, max_m, k // 128), 1.0, np.float32)
    for e in range(e_n):
        r0, r1 = int(offsets[e]), int(offsets[e + 1])
        a3[e, :r1 - r0] = aq[r0:r1]
        s3[e, :r1 - r0] = as_[r0:r1]
    return a3, s3


@pytest.mark.gpu
@pytest.mark.parametrize("name", GROUPED)
def test_grouped_masked_layout(name):
    # every expert owns max_m rows of which counts[e] are valid: the valid rows
    # equal the contiguous layout's bit for bit (same configuration, same rows
    # counted from the segment start) and the oracle; rows past a count keep
    # their contents
    device()
    counts = [5, 0, 64, 1, 37, 64, 20, 0]
    max_m, n, k = 64, 392, 768
    aq, as_, bq, bs, offsets = _experts(counts, n, k, seed=17)
    a3, s3 = _masked_inputs(counts, max_m, aq, as_, offsets)
    m = int(offsets[-1])
    cfg = _cfg(name)
    B, BS = to_dev(bq), to_dev(bs)
    for out in ("bf16", "fp32"):
        flat = _grouped(to_dev(aq), to_dev(as_), B, BS, to_dev(offsets), m, n, k, out, cfg)
        c3 = torch.full((len(counts), max_m, n), float("nan"), dtype=TORCH_OUT[out],
                        device="cuda:0")
        st = inferop_amd.w8a8_block_fp8_grouped_gemm_masked_config(
            c3, to_dev(a3), to_dev(s3), B, BS, to_dev(np.array(counts, np.int32)), max_m, n, k,
            len(counts), getattr(DT, out), cfg)
        assert st == 0
        for e, cnt in enumerate(counts):
            r0 = int(offsets[e])
            assert torch.equal(c3[e, :cnt], flat[r0:r0 + cnt]), f"{name} {out} expert {e}"
            assert torch.isnan(c3[e, cnt:].float()).all(), f"{name} {out} expert {e} tail"
            if cnt:
                assert_gemm_close(out_to_f32(c3[e, :cnt]),
                                  oracle.gemm(aq[r0:r0 + cnt], as_[r0:r0 + cnt], bq[e], bs[e]),
                                  f"{name} {out} expert {e}")


@pytest.mark.gpu
def test_grouped_masked_counts_clamped_and_hint():
    # counts are device data: negative counts act as 0 and counts past max_m
    # as max_m; expected_m only steers the tile choice (the result is the same
    # within the tolerance whatever the hint)
    device()
    counts = [-3, 40, 1000, 7]
    eff = [0, 32, 32, 7]
    max_m, n, k = 32, 256, 512
    aq, as_, bq, bs, offsets = _experts(eff, n, k, seed=29)
    a3, s3 = _masked_inputs(eff, max_m, aq, as_, offsets)
    args = [to_dev(v) for v in (a3, s3, bq, bs, np.array(counts, np.int32))]
    for hint in (0, 2, 20, 500):
        c3 = torch.full((len(counts), max_m, n), float("nan"), device="cuda:0")
        assert inferop_amd.w8a8_block_fp8_grouped_gemm_masked(
            c3, *args, max_m, n, k, len(counts), hint, out_dt=DT.fp32) == 0
        got = out_to_f32(c3)
        assert np.isnan(got[0]).all()
        for e in (1, 2, 3):
            r0, cnt = int(offsets[e]), eff[e]
            assert_gemm_close(got[e, :cnt], oracle.gemm(aq[r0:r0 + cnt], as_[r0:r0 + cnt], bq[e],
                                                         bs[e]), f"hint {hint} expert {e}")
            assert np.isnan(got[e, cnt:]).all()
