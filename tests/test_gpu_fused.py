"""Producers fused with the per-token-group quantizer against the oracle.

The unfused reference flow is silu_and_mul / fused_add_rmsnorm writing dt
(reference.cpp:23-35, 55-64 for the arithmetic; the stored value is the
round-to-nearest-even dt conversion the reference kernels use), then
quant_fp8_per_token_group on that dt tensor (reference.cpp:65-80).  The oracle
side composes exactly that.  SiLU: exp is evaluated on the device in double
precision and rounded once, the C library's expf on the host; both are
correctly rounded except in rare last-bit cases, so the bf16 / fp16 tests run
every finite gate value and allow at most 1 differing byte in 10^4.  RMSNorm:
the device sums squares as a tree, the reference left to right; inputs whose
partial sums are exact give bit-exact bytes, normal inputs are compared
within one E4M3 step."""
import numpy as np
import pytest
import torch

import inferop_amd as ia
import oracle
from datagen import bf16_bits_to_f32, f32_to_bf16_bits
from gpu_util import bf16_dev, device, f16_dev, to_dev

pytestmark = pytest.mark.gpu
DT = ia.dtype


def _round_dt(x32: np.ndarray, kind: str) -> np.ndarray:
    """fp32 value of the nearest-even dt rounding (the device stores)."""
    if kind == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x32))
    if kind == "fp16":
        with np.errstate(over="ignore"):
            return x32.astype(np.float16).astype(np.float32)
    return x32.astype(np.float32)


def _dev(x32: np.ndarray, kind: str):
    """Device tensor holding the dt rounding of x32, and those values in fp32."""
    xr = _round_dt(x32, kind)
    if kind == "bf16":
        return bf16_dev(f32_to_bf16_bits(xr)), xr
    if kind == "fp16":
        return f16_dev(xr.astype(np.float16).view(np.uint16)), xr
    return to_dev(xr), xr


def _silu_gpu(gu_dev, kind, tokens, d):
    q = torch.full((tokens, d), 0xA5, dtype=torch.uint8, device="cuda:0")
    s = torch.full((tokens, d // 128), -1.0, dtype=torch.float32, device="cuda:0")
    st = ia.silu_and_mul_quant_fp8(q, s, gu_dev, getattr(DT, kind), tokens, d)
    assert st == 0, st
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


def _silu_oracle(gu32, kind):
    y = _round_dt(oracle.silu_and_mul(gu32), kind)
    return oracle.quant(y)


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_silu_quant_every_gate_value(kind):
    device()
    # every finite 16-bit gate pattern, twice: up = 1 and up = a normal draw
    if kind == "bf16":
        bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
        vals = bf16_bits_to_f32(bits)
    else:
        vals = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    vals = vals[np.isfinite(vals)]
    d = 1024
    n = (len(vals) // d) * d
    # repeated 40 times in shifted order: 19840 (fp16) / 20160 (bf16)
    # groups, enough for the kernel that copies its SiLU tables into LDS (64
    # groups per CU: 16384 on 256 CUs)
    gate = np.concatenate([np.roll(vals[:n], 97 * r) for r in range(40)]).reshape(-1, d)
    tokens = gate.shape[0]
    g = np.random.default_rng(31)
    for up in (np.ones_like(gate), g.standard_normal(gate.shape).astype(np.float32)):
        gu32 = np.concatenate([gate, up], axis=1)
        gu_dev, gu_exact = _dev(gu32, kind)
        q, s = _silu_gpu(gu_dev, kind, tokens, d)
        qr, sr = _silu_oracle(gu_exact, kind)
        bad_s = int((s.view(np.uint32) != sr.view(np.uint32)).sum())
        bad_q = int((q != qr).sum())
        assert bad_q <= q.size // 10000 and bad_s <= s.size // 1000, (bad_q, bad_s)


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_silu_lds_tables_match_small_call_kernel(kind):
    # 32768 tokens x 128 outputs = 32768 groups take the kernel that holds
    # a slice of its SiLU table in LDS (it needs 64 groups per CU: 16384 on
    # 256 CUs) and gathers the other patterns from the full table; 512-token
    # calls take the kernel that gathers from the full bf16 table or
    # evaluates the SiLU for fp16.  Rows are independent, so both must give
    # the same bits for every 16-bit gate pattern, Inf and NaN included (the
    # tables hold the same arithmetic's results).
    device()
    tokens, d = 32768, 128
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    reps = -(-tokens * d // 65536)
    gate = np.concatenate([np.roll(pats, 131 * r) for r in range(reps)])[: tokens * d]
    g = np.random.default_rng(8200)
    up32 = (2.0 * g.standard_normal(tokens * d)).astype(np.float32)
    up = f32_to_bf16_bits(up32) if kind == "bf16" else up32.astype(np.float16).view(np.uint16)
    gu = np.ascontiguousarray(np.concatenate([gate.reshape(tokens, d), up.reshape(tokens, d)], axis=1))
    gu_dev = bf16_dev(gu) if kind == "bf16" else f16_dev(gu)
    q, s = _silu_gpu(gu_dev, kind, tokens, d)
    for r0 in range(0, tokens, 512):
        r1 = min(tokens, r0 + 512)
        qs, ss = _silu_gpu(gu_dev[r0:r1].contiguous(), kind, r1 - r0, d)
        assert np.array_equal(qs, q[r0:r1]), r0
        assert np.array_equal(ss.view(np.uint32), s[r0:r1].view(np.uint32)), r0


@pytest.mark.parametrize("kind", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("shape", [(1, 2048), (64, 18432 // 8), (77, 7168 // 4), (16411, 128),
                                   (4096, 18432 // 8)])
def test_silu_quant_parity(kind, shape):
    device()
    tokens, d = shape
    g = np.random.default_rng(tokens + d)
    gu32 = (2.0 * g.standard_normal((tokens, 2 * d))).astype(np.float32)
    gu_dev, gu_exact = _dev(gu32, kind)
    q, s = _silu_gpu(gu_dev, kind, tokens, d)
    qr, sr = _silu_oracle(gu_exact, kind)
    assert int((q != qr).sum()) <= max(1, q.size // 10000)
    assert int((s.view(np.uint32) != sr.view(np.uint32)).sum()) <= max(1, s.size // 1000)
    # every scale within an ulp of the oracle's, every byte within one code
    assert np.allclose(s, sr, rtol=2.0 ** -22, atol=0)
    assert (np.abs(q.astype(np.int16) - qr.astype(np.int16)) <= 1).all()


def _rms_gpu(res_dev, x_dev, w_dev, kind, rows, cols, eps):
    q = torch.full((rows, cols), 0xA5, dtype=torch.uint8, device="cuda:0")
    s = torch.full((rows, cols // 128), -1.0, dtype=torch.float32, device="cuda:0")
    st = ia.fused_add_rmsnorm_quant_fp8(res_dev, q, s, x_dev, w_dev, getattr(DT, kind), rows,
                                        cols, eps)
    assert st == 0, st
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


def _rms_oracle(res, x, w, kind, eps):
    r_new = _round_dt(res + x, kind)               # the stored residual
    y = _round_dt(oracle.rmsnorm(r_new, w, eps), kind)
    q, s = oracle.quant(y)
    return r_new, q, s


def _res_values(res_dev, kind):
    t = res_dev.detach()
    if kind == "bf16":
        return bf16_bits_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))
    return t.float().cpu().numpy()


@pytest.mark.parametrize("kind", ["bf16", "fp16", "fp32"])
def test_add_rmsnorm_quant_exact_sums(kind):
    # small integers: every square and partial sum is exact in fp32, so the
    # summation order cannot matter and the bytes must agree exactly
    device()
    rows, cols = 37, 7168
    g = np.random.default_rng(41)
    res = g.integers(-6, 7, (rows, cols)).astype(np.float32)
    x = g.integers(-6, 7, (rows, cols)).astype(np.float32)
    w = (g.integers(1, 9, cols) / 8).astype(np.float32)
    rd, rexact = _dev(res, kind)
    xd, xexact = _dev(x, kind)
    wd, wexact = _dev(w, kind)
    q, s = _rms_gpu(rd, xd, wd, kind, rows, cols, 1e-6)
    r_new, qr, sr = _rms_oracle(rexact, xexact, wexact, kind, 1e-6)
    assert np.array_equal(_res_values(rd, kind).view(np.uint32), r_new.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))
    assert np.array_equal(q, qr)


@pytest.mark.parametrize("kind", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("shape", [(1, 7168), (64, 7168), (16, 18432), (5, 128)])
def test_add_rmsnorm_quant_normal_inputs(kind, shape):
    device()
    rows, cols = shape
    g = np.random.default_rng(rows * 7 + cols)
    res = g.standard_normal((rows, cols)).astype(np.float32)
    x = (0.5 * g.standard_normal((rows, cols))).astype(np.float32)
    w = (1.0 + 0.1 * g.standard_normal(cols)).astype(np.float32)
    rd, rexact = _dev(res, kind)
    xd, xexact = _dev(x, kind)
    wd, wexact = _dev(w, kind)
    q, s = _rms_gpu(rd, xd, wd, kind, rows, cols, 1e-6)
    r_new, qr, sr = _rms_oracle(rexact, xexact, wexact, kind, 1e-6)
    # the residual update is one rounding of res + x: exact
    assert np.array_equal(_res_values(rd, kind).view(np.uint32), r_new.view(np.uint32))
    # The inverse RMS differs by the reference's left-to-right summation error
    # (at most about cols * 2^-24 relative, all terms being positive).  After
    # the dt rounding that moves a group's absmax by at most one dt ulp, so a
    # few groups' scales differ by up to one ulp of dt; the others must agree
    # bit for bit with every byte within one E4M3 code.
    ulp = {"bf16": 2.0 ** -7, "fp16": 2.0 ** -10, "fp32": (cols + 8) * 2.0 ** -24}[kind]
    assert np.allclose(s, sr, rtol=ulp, atol=0)
    same = s.view(np.uint32) == sr.view(np.uint32)
    if kind == "fp32":  # no dt rounding to absorb the difference: compare all groups
        same[:] = True
    assert same.mean() >= 0.99
    qg, qrg = q.reshape(rows, -1, 128), qr.reshape(rows, -1, 128)
    assert (np.abs(qg[same].astype(np.int16) - qrg[same].astype(np.int16)) <= 1).all()
    assert int((qg[same] != qrg[same]).sum()) <= max(2, q.size // 1000)
    # every group: the dequantized output within E4M3 precision of the
    # oracle's dt output
    y_ref = _round_dt(oracle.rmsnorm(r_new, wexact, 1e-6), kind)
    deq = oracle.e4m3_decode_table()[q] * np.repeat(s, 128, axis=1)
    assert (np.abs(deq - y_ref) <= 0.07 * np.abs(y_ref) + np.repeat(s, 128, axis=1) * 2.0 ** -8).all()


def test_fused_rejected_calls():
    device()
    S = ia.Status
    gu = torch.zeros((4, 512), dtype=torch.bfloat16, device="cuda:0")
    q = torch.full((4, 256), 0xAB, dtype=torch.uint8, device="cuda:0")
    s = torch.full((4, 2), 7.0, dtype=torch.float32, device="cuda:0")
    f = ia.silu_and_mul_quant_fp8
    assert f(q, s, gu, DT.bf16, 4, 200) == S.ERR_SHAPE
    assert f(q, s, gu, DT.bf16, 4, 256, group_size=64) == S.ERR_SHAPE
    assert f(q, s, gu, DT.fp8_e4m3, 4, 256) == S.ERR_DTYPE
    assert f(q, s, gu.data_ptr() + 2, DT.bf16, 2, 128) == S.ERR_ARGUMENT
    r = torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda:0")
    h = ia.fused_add_rmsnorm_quant_fp8
    assert h(r, q, s, r, r[0], DT.bf16, 4, 200) == S.ERR_SHAPE
    assert h(r, q, s, r, r[0], DT.fp8_e4m3, 4, 256) == S.ERR_DTYPE
    assert h(r, q, s, r, r.data_ptr() + 2, DT.bf16, 4, 256) == S.ERR_ARGUMENT
    torch.cuda.synchronize()
    assert (q == 0xAB).all() and (s == 7.0).all()
