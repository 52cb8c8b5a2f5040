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
