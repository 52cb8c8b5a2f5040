"""GPU weight block quantizer (the reference's GEMM-test weight recipe,
tests/test_gemm.cpp:28-45) against the oracle: bytes and scales bit-exact for
fp32 / bf16 / fp16 weights, ragged N, outlier blocks and special values, and
the GEMM fed with GPU-quantized weights."""
import numpy as np
import pytest

import oracle
from datagen import (bf16_bits_to_f32, f16_bits_to_f32, f32_to_bf16_bits, f32_to_f16_bits,
                     weights)
import torch

import inferop_amd as ia
from gpu_util import assert_gemm_close, bf16_dev, device, f16_dev, to_dev

pytestmark = pytest.mark.gpu


def _to_device(w32: np.ndarray, kind: str):
    """Exact `kind` values of w32 on the device, and their fp32 values."""
    device()
    if kind == "fp32":
        return to_dev(w32), w32
    if kind == "bf16":
        bits = f32_to_bf16_bits(w32)
        return bf16_dev(bits), bf16_bits_to_f32(bits)
    bits = f32_to_f16_bits(w32)
    return f16_dev(bits), f16_bits_to_f32(bits)


def _check(w32: np.ndarray, kind: str):
    wt, wexact = _to_device(w32, kind)
    q, s = ia.quantize_weight(wt)
    torch.cuda.synchronize()
    qr, sr = oracle.weight_block_quant(wexact)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), sr.view(np.uint32))
    got = q.cpu().numpy()
    bad = np.argwhere(got != qr)
    assert bad.size == 0, f"{len(bad)} bytes differ, first at {bad[0]}: {got[tuple(bad[0])]:#x} vs {qr[tuple(bad[0])]:#x}"


@pytest.mark.parametrize("kind", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("shape", [(512, 1024), (4672, 1024), (77, 384), (128, 128)])
def test_weight_quant_parity(kind, shape):
    n, k = shape
    _check(weights(n, k, 11, "stress"), kind)


@pytest.mark.parametrize("kind", ["fp32", "bf16", "fp16"])
def test_weight_quant_special_blocks(kind):
    g = np.random.default_rng(5)
    w = (0.02 * g.standard_normal((256, 128 * 10))).astype(np.float32)
    w[:, 0:128] = 0.0                                   # zero block -> scale 1
    w[3, 128 + 5] = np.nan                              # NaN ignored by absmax
    w[7, 256 + 9] = np.inf                              # Inf block
    w[130, 384 + 1] = -np.inf
    w[131, 384 + 2] = np.nan
    w[:, 512:640] *= np.float32(2.0 ** -90)             # absmax below 2^-80: slow path
    w[:, 640:768] *= np.float32(2.0 ** -80)             # at the threshold
    w[:, 768:896] = -0.0
    w[200, 896:1024] = 1e4                              # one outlier row
    if kind == "fp32":
        w[:, 1024:1152] *= np.float32(2.0 ** -120)      # fp32 subnormal inputs
    w[129, 1152 + 3] = -np.nan
    _check(w, kind)


def test_weight_quant_rejected_calls():
    S = ia.Status
    w = torch.zeros((128, 256), dtype=torch.float32, device=device())
    q = torch.full((128, 256), 0xAB, dtype=torch.uint8, device=device())
    s = torch.full((1, 2), 7.0, dtype=torch.float32, device=device())
    f = ia.quant_fp8_weight_block
    assert f(q, s, w, ia.dtype.fp32, 128, 250) == S.ERR_SHAPE
    assert f(q, s, w, ia.dtype.fp32, 128, 256, group_size=64) == S.ERR_SHAPE
    assert f(q, s, w, ia.dtype.fp32, 128, 256, block_n=64) == S.ERR_SHAPE
    assert f(q, s, w, ia.dtype.fp8_e4m3, 128, 256) == S.ERR_DTYPE
    assert f(q, s, w.data_ptr() + 4, ia.dtype.fp32, 64, 128) == S.ERR_ARGUMENT
    torch.cuda.synchronize()
    assert (q == 0xAB).all() and (s == 7.0).all()


def test_gemm_on_gpu_quantized_weights():
    m, n, k = 64, 2112, 1024
    g = np.random.default_rng(3)
    a32 = g.standard_normal((m, k), dtype=np.float32)
    bits = f32_to_bf16_bits(a32)
    a = torch.from_numpy(bits.view(np.int16)).to(device()).view(torch.bfloat16)
    wt = torch.from_numpy(weights(n, k, 4, "normal")).to(device())
    aq, as_ = ia.quantize(a)
    bq, bs = ia.quantize_weight(wt)
    c = ia.gemm(aq, as_, bq, bs, out_dtype=torch.float32)
    torch.cuda.synchronize()
    qr, sr = oracle.quant(bf16_bits_to_f32(bits))
    bqr, bsr = oracle.weight_block_quant(weights(n, k, 4, "normal"))
    assert np.array_equal(bq.cpu().numpy(), bqr)
    ref = oracle.gemm(qr, sr, bqr, bsr)
    assert_gemm_close(c.cpu().numpy(), ref, "gpu-quantized weights")
