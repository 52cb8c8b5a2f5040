"""The quantizer and the GEMM in one call (inferop_quant_w8a8_block_fp8_gemm,
no counterpart in the reference: its decode step is quant_fp8_per_token_group,
ops.h:64-65, then w8a8_block_fp8_gemm, ops.h:81-84).  It must write the very
bytes the two calls write: q / scales equal to the quantizer's (and so to the
oracle's, reference.cpp:65-80) and C equal bit for bit to the GEMM on them --
on every configs[1] shape (one launch at M = 1, two at M = 16 and 64), on
fp16 and fp32 activations, ragged N, and the quantizer's edge groups (NaN,
Inf, zero, subnormal) -- and C within the GEMM tolerance of the oracle."""
import numpy as np
import pytest
import torch

import datagen
import inferop_amd
import oracle
from gpu_util import assert_gemm_close, device, to_dev, to_np

DT = inferop_amd.dtype
TORCH_IN = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _x_dev(x32, kind):
    """fp32 values exactly representable in `kind` -> device tensor of that dtype."""
    if kind == "bf16":
        return to_dev(datagen.f32_to_bf16_bits(x32)).view(torch.bfloat16)
    if kind == "fp16":
        return to_dev(datagen.f32_to_f16_bits(x32)).view(torch.float16)
    return to_dev(x32.astype(np.float32))


def _run_both(x, kind, bq, bs, m, n, k, out=torch.bfloat16):
    """(q, s, c) of the one-call path and of the two calls, on the GPU."""
    odt = {torch.bfloat16: DT.bf16, torch.float16: DT.fp16, torch.float32: DT.fp32}[out]
    dev = "cuda:0"
    q1 = torch.full((m, k), 0x5A, dtype=torch.uint8, device=dev)
    s1 = torch.full((m, k // 128), -1.0, dtype=torch.float32, device=dev)
    c1 = torch.full((m, n), float("nan"), dtype=out, device=dev)
    assert inferop_amd.quant_w8a8_block_fp8_gemm(c1, q1, s1, x, getattr(DT, kind), bq, bs, m, n,
                                                 k, out_dt=odt) == 0
    q2 = torch.empty_like(q1)
    s2 = torch.empty_like(s1)
    c2 = torch.full((m, n), float("nan"), dtype=out, device=dev)
    assert inferop_amd.quant_fp8_per_token_group(q2, s2, x, getattr(DT, kind), m, k) == 0
    assert inferop_amd.w8a8_block_fp8_gemm(c2, q2, s2, bq, bs, m, n, k, out_dt=odt) == 0
    torch.cuda.synchronize()
    return (q1, s1, c1), (q2, s2, c2)


def _same_bits(a, b):
    if a.dtype in (torch.bfloat16, torch.float16):
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 16, 64])
@pytest.mark.parametrize("nk", [(7168, 2048), (4096, 7168), (2112, 7168)])
def test_config1_quant_gemm_matches_two_calls(m, nk):
    device()
    n, k = nk
    launches = inferop_amd.quant_gemm_launches(m, n, k)
    print(f"quant+gemm m={m} n={n} k={k} launches={launches}", flush=True)
    assert launches == (1 if m == 1 else 2)
    a_bits, a_f32, bq, bs = datagen.gemm_case(m, n, k, seed=100 + m)
    x = to_dev(a_bits).view(torch.bfloat16)
    (q1, s1, c1), (q2, s2, c2) = _run_both(x, "bf16", to_dev(bq), to_dev(bs), m, n, k)
    qr, sr = oracle.quant(a_f32)
    assert np.array_equal(to_np(q1), qr)
    assert np.array_equal(to_np(s1).view(np.uint32), sr.view(np.uint32))
    assert _same_bits(q1, q2) and _same_bits(s1, s2)
    assert _same_bits(c1, c2), "C differs from the two-call path"
    assert_gemm_close(c1.float().cpu().numpy(), oracle.gemm(qr, sr, bq, bs),
                      f"quant+gemm {m}x{n}x{k}")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("m,n,k", [(1, 1000, 1024), (3, 4096, 7168), (5, 2112, 2048),
                                   (8, 512, 8192), (2, 7168, 7168), (7, 300, 128)])
def test_fused_rows_dtypes_and_ragged_n(kind, m, n, k):
    device()
    print(f"quant+gemm {kind} m={m} n={n} k={k} "
          f"launches={inferop_amd.quant_gemm_launches(m, n, k)}", flush=True)
    x32 = datagen.activations(m, k, 7 + m, "stress")
    if kind == "bf16":
        x32 = datagen.bf16_bits_to_f32(datagen.f32_to_bf16_bits(x32))
    elif kind == "fp16":
        x32 = datagen.f16_bits_to_f32(datagen.f32_to_f16_bits(x32))
    bq, bs = oracle.weight_block_quant(datagen.weights(n, k, 8 + n))
    for out in (torch.bfloat16, torch.float32):
        (q1, s1, c1), (q2, s2, c2) = _run_both(_x_dev(x32, kind), kind, to_dev(bq), to_dev(bs), m,
                                               n, k, out)
        qr, sr = oracle.quant(x32)
        assert np.array_equal(to_np(q1), qr)
        assert np.array_equal(to_np(s1).view(np.uint32), sr.view(np.uint32))
        assert _same_bits(c1, c2)
        assert_gemm_close(c1.float().cpu().numpy(), oracle.gemm(qr, sr, bq, bs), f"{kind} {m}")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["bf16", "fp16", "fp32"])
def test_fused_edge_groups(kind):
    # the quantizer's edge groups (zero, -0, NaN, Inf, subnormal, tiny, huge)
    # spread over 8 rows x 16 groups: codes and scales equal the oracle's and
    # C (NaN where an input group is NaN or Inf) equals the two-call path bit
    # for bit
    device()
    m, n, k = 8, 640, 2048
    rows = datagen.special_groups(kind)
    groups = [rows[i % len(rows)] for i in range(m * (k // 128))]
    x32 = np.concatenate(groups).reshape(m, k).astype(np.float32)
    bq, bs = oracle.weight_block_quant(datagen.weights(n, k, 3))
    assert inferop_amd.quant_gemm_launches(m, n, k) == 1
    (q1, s1, c1), (q2, s2, c2) = _run_both(_x_dev(x32, kind), kind, to_dev(bq), to_dev(bs), m, n,
                                           k, torch.float32)
    qr, sr = oracle.quant(x32)
    assert np.array_equal(to_np(q1), qr)
    assert np.array_equal(to_np(s1).view(np.uint32), sr.view(np.uint32))
    assert _same_bits(c1, c2)


@pytest.mark.gpu
def test_fused_graph_replays_and_unaligned_input():
    device()
    m, n, k = 1, 2112, 7168
    a_bits, a_f32, bq, bs = datagen.gemm_case(m, n, k, seed=21)
    x = to_dev(a_bits).view(torch.bfloat16)
    bqd, bsd = to_dev(bq), to_dev(bs)
    st = torch.cuda.Stream()
    q = torch.empty((m, k), dtype=torch.uint8, device="cuda:0")
    s = torch.empty((m, k // 128), dtype=torch.float32, device="cuda:0")
    c = torch.empty((m, n), dtype=torch.bfloat16, device="cuda:0")

    def call():
        assert inferop_amd.quant_w8a8_block_fp8_gemm(c, q, s, x, DT.bf16, bqd, bsd, m, n, k,
                                                     stream=st.cuda_stream) == 0

    with torch.cuda.stream(st):
        call()
    st.synchronize()
    want = (q.clone(), s.clone(), c.clone())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        call()
    for rep in range(3):
        q.zero_()
        s.zero_()
        c.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert all(_same_bits(a, b) for a, b in zip((q, s, c), want)), f"replay {rep}"
    # x at a 2-byte offset: not 16-byte aligned, so the two-launch path; same bytes
    buf = torch.empty(m * k + 8, dtype=torch.bfloat16, device="cuda:0")
    buf[1:1 + m * k] = x.view(-1)
    xu = buf[1:1 + m * k].view(m, k)
    q2 = torch.empty_like(q)
    s2 = torch.empty_like(s)
    c2 = torch.empty_like(c)
    assert inferop_amd.quant_w8a8_block_fp8_gemm(c2, q2, s2, xu, DT.bf16, bqd, bsd, m, n, k) == 0
    torch.cuda.synchronize()
    assert _same_bits(q2, want[0]) and _same_bits(s2, want[1]) and _same_bits(c2, want[2])


@pytest.mark.gpu
def test_fused_guards():
    device()
    S = inferop_amd.Status
    z = torch.zeros(4096, dtype=torch.uint8, device="cuda:0")
    c = torch.full((2, 16), 3.0, dtype=torch.float32, device="cuda:0")
    f = inferop_amd.quant_w8a8_block_fp8_gemm
    assert f(c, z, z, z, DT.bf16, z, z, 2, 16, 100) == S.ERR_SHAPE
    assert f(c, z, z, z, DT.bf16, z, z, 2, 16, 128, group_size=64) == S.ERR_SHAPE
    assert f(c, z, z, z, DT.fp8_e4m3, z, z, 2, 16, 128) == S.ERR_DTYPE
    assert f(c, z, z, z, DT.bf16, z, z, 2, 16, 128, out_dt=DT.fp8_e4m3) == S.ERR_DTYPE
    torch.cuda.synchronize()
    assert (c == 3.0).all()
