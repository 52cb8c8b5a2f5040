"""Helpers for the GPU parity tests (device buffers through torch, tolerance)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import inferop_amd


def device():
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    inferop_amd.lib()  # raises if libinferop.so is missing: no fallback
    assert inferop_amd.has_cuda()
    return torch.device("cuda:0")


def to_dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to("cuda:0")
    return torch.from_numpy(a).to("cuda:0")


def bf16_dev(bits: np.ndarray) -> torch.Tensor:
    return to_dev(bits).view(torch.bfloat16)


def f16_dev(bits: np.ndarray) -> torch.Tensor:
    return to_dev(bits).view(torch.float16)


def to_np(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    if t.dtype == torch.float16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def out_to_f32(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    a = np.abs(v.astype(np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def assert_gemm_close(got: np.ndarray, ref: np.ndarray, what: str = ""):
    """max |got - ref| <= 1e-2 * rms(ref) + one bf16 ulp of |ref| (elementwise),
    the tolerance BASELINE.json states for the blockwise GEMM."""
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    assert got.shape == ref.shape
    assert np.isfinite(got).all(), what
    rms = np.sqrt(np.mean(ref ** 2))
    tol = 1e-2 * rms + bf16_ulp(ref)
    err = np.abs(got - ref)
    bad = err > tol
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{bad.size} out of tolerance, "
                           f"max excess {float((err - tol).max()):.3g}, rms {rms:.3g}")
    return float(err.max() / rms) if rms > 0 else 0.0


def gemm_ref_f64(aq: torch.Tensor, as_: torch.Tensor, bq: torch.Tensor,
                 bs: torch.Tensor) -> torch.Tensor:
    """The GEMM oracle's sum (reference.cpp:93-110) as one float64 matmul on
    the GPU: operands dequantized exactly as the reference does -- the E4M3
    value times its fp32 scale, rounded to fp32 -- then widened to float64;
    only the order of the float64 additions differs from the oracle's, which
    moves a result by far less than one fp32 ulp (checked against the oracle
    on sampled rows by anchor_ref_rows).  Returns C [M, N] float64."""
    m, k = aq.shape
    n = bq.shape[0]
    kg = k // 128
    a = aq.view(torch.float8_e4m3fn).float().view(m, kg, 128) * as_.view(m, kg, 1)
    sb = bs.repeat_interleave(128, dim=0)[:n]
    b = bq.view(torch.float8_e4m3fn).float().view(n, kg, 128) * sb.view(n, kg, 1)
    a64 = a.view(m, k).double()
    del a
    b64t = b.view(n, k).double().t().contiguous()
    del b
    return torch.mm(a64, b64t)


def anchor_ref_rows(ref: torch.Tensor, want_rows: np.ndarray, rows: np.ndarray, what: str = ""):
    """The float64 GPU reference agrees with the oracle's fp32 outputs on the
    sampled rows to within one fp32 ulp (the oracle rounds its float64 sum to
    fp32 once): a wrong dequantization (scale index, transposed operand,
    dropped group) would fail here."""
    got = ref[torch.as_tensor(rows, device=ref.device)].cpu().numpy()
    want = want_rows.astype(np.float64)
    ulp = np.spacing(np.abs(want_rows.astype(np.float32))).astype(np.float64)
    bad = np.abs(got - want) > ulp
    assert not bad.any(), (f"{what}: float64 reference differs from the oracle on "
                           f"{int(bad.sum())}/{bad.size} sampled outputs")


def assert_gemm_close_dev(got: torch.Tensor, ref: torch.Tensor, what: str = ""):
    """assert_gemm_close over every element, on the GPU: got (any float dtype,
    prefilled with NaN by the caller so an unwritten element fails) against
    the float64 reference."""
    g = got.double()
    assert g.shape == ref.shape
    finite = torch.isfinite(g)
    assert bool(finite.all()), f"{what}: {int((~finite).sum())} outputs NaN/Inf (unwritten?)"
    rms = torch.sqrt(torch.mean(ref * ref))
    ulp = torch.exp2(torch.floor(torch.log2(torch.clamp(ref.abs(), min=2.0 ** -126))) - 7)
    tol = 1e-2 * rms + ulp
    err = (g - ref).abs()
    bad = err > tol
    nbad = int(bad.sum())
    assert nbad == 0, (f"{what}: {nbad}/{bad.numel()} out of tolerance, "
                       f"max excess {float((err - tol).max()):.3g}, rms {float(rms):.3g}")
    return float(err.max() / rms) if float(rms) > 0 else 0.0
