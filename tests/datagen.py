"""Seeded synthetic inputs for the FP8 path (tests and fixture generation).

numpy's PCG64 generator keyed by ``seed`` (independent of call order), so a
case can be regenerated exactly on any host.  Activations are produced as
bf16 / fp16 bit patterns with the reference's host conversions
(include/inferop/common.h:57-61, 80-101) plus their exact fp32 values, which
is what the CPU oracle must be fed (identical inputs on both sides).
"""
from __future__ import annotations

import numpy as np

import oracle


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """common.h:57-61 float_to_bf16_rn, vectorised."""
    w = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((w + 0x7FFF + ((w >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """common.h:80-101 float_to_half_rn via the oracle (exact restatement)."""
    x = np.ascontiguousarray(x, np.float32)
    L = oracle.lib()
    out = np.empty(x.size, np.uint16)
    flat = x.reshape(-1)
    # numpy's IEEE conversion agrees with the reference except for the two
    # documented departures, which are patched below.
    h = flat.astype(np.float16).view(np.uint16).copy()
    a = np.abs(flat)
    big = (a > 65504.0) & np.isfinite(flat)
    h[big] = np.where(np.signbit(flat[big]), 0xFC00, 0x7C00)
    small = (a < np.float32(2.0 ** -24)) & (a > 0)
    h[small] = np.where(np.signbit(flat[small]), 0x8000, 0x0000)
    h[np.isnan(flat)] = 0x7E00
    out[:] = h
    del L
    return out.reshape(x.shape)


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return np.asarray(b, np.uint16).view(np.float16).astype(np.float32)


def rng(seed: int, stream: int = 0) -> np.random.Generator:
    return np.random.default_rng([seed, stream])


def activations(m: int, k: int, seed: int, dist: str = "normal") -> np.ndarray:
    """fp32 activations before 16-bit packing.

    normal: N(0, 1).  stress (config 4): 4 * Student-t(3), 1% of 1x128 groups
    set to zero, 0.1% of elements set to +-1792 (= 448 * 4, the largest
    outliers the scaled distribution is quoted with)."""
    g = rng(seed, 1)
    if dist == "normal":
        return g.standard_normal((m, k), dtype=np.float32)
    if dist == "stress":
        x = (4.0 * g.standard_t(3, size=(m, k))).astype(np.float32)
        kg = k // 128
        groups = x[:, :kg * 128].reshape(m, kg, 128)
        zero = g.random((m, kg)) < 0.01
        groups[zero] = 0.0
        x[:, :kg * 128] = groups.reshape(m, kg * 128)
        out = g.random((m, k)) < 0.001
        sign = np.where(g.random((m, k)) < 0.5, -1.0, 1.0).astype(np.float32)
        x[out] = 1792.0 * sign[out]
        return x
    raise ValueError(dist)


def weights(n: int, k: int, seed: int, dist: str = "normal") -> np.ndarray:
    """fp32 weights N(0, 0.02); stress: 1% of 128x128 blocks scaled x100."""
    g = rng(seed, 2)
    w = (0.02 * g.standard_normal((n, k), dtype=np.float32)).astype(np.float32)
    if dist == "stress":
        nb, kb = (n + 127) // 128, k // 128
        hot = np.argwhere(g.random((nb, kb)) < 0.01)
        for bn, bk in hot:
            w[bn * 128:(bn + 1) * 128, bk * 128:(bk + 1) * 128] *= 100.0
    return w


def gemm_case(m: int, n: int, k: int, seed: int, dist: str = "normal"):
    """bf16 activations (bits + exact fp32) and block-quantized weights."""
    a32 = activations(m, k, seed, dist)
    a_bits = f32_to_bf16_bits(a32)
    a_f32 = bf16_bits_to_f32(a_bits)
    bq, bs = oracle.weight_block_quant(weights(n, k, seed, dist))
    return a_bits, a_f32, bq, bs


def special_groups(kind: str = "bf16") -> np.ndarray:
    """fp32 rows of 128-element groups covering the quantizer's edge cases,
    each value exactly representable in `kind` (bf16 / fp16 / fp32)."""
    g = rng(1234, 3)
    rows = []
    base = g.standard_normal(128).astype(np.float32)
    rows.append(np.zeros(128, np.float32))                         # zero group -> scale 1
    rows.append(-np.zeros(128, np.float32))                        # all -0
    r = base.copy(); r[::7] = -0.0; rows.append(r)                 # -0 inside a normal group
    r = base.copy(); r[5] = np.nan; rows.append(r)                 # NaN ignored by absmax
    r = base.copy(); r[9] = -np.nan; rows.append(r)
    r = base.copy(); r[3] = np.inf; rows.append(r)                 # Inf: scale Inf
    r = base.copy(); r[3] = -np.inf; r[4] = np.inf; rows.append(r)
    r = np.zeros(128, np.float32); r[0] = np.nan; rows.append(r)   # NaN in a zero group
    r = base * np.float32(2.0 ** -20); rows.append(r)              # small normal
    r = base * np.float32(448.0); rows.append(r)
    r = np.full(128, 448.0, np.float32); r[1::2] = -448.0; rows.append(r)
    r = base.copy(); r[0] = 1e4; rows.append(r)                    # one outlier
    if kind == "bf16":
        r = base * np.float32(2.0 ** -90); rows.append(r)         # absmax < 2^-80: slow path
        r = base * np.float32(2.0 ** -128); rows.append(r)        # bf16 subnormals
        r = base * np.float32(2.0 ** -135); rows.append(r)        # scale underflows to 0
        r = base / np.abs(base).max() * np.float32(3.0e38); rows.append(r)  # near bf16 max
        r = base * np.float32(2.0 ** -80); rows.append(r)         # at the threshold
    elif kind == "fp16":
        r = base * np.float32(2.0 ** -16); rows.append(r)         # fp16 subnormals
        r = base * np.float32(60000.0 / 4.0); rows.append(r)
        r = np.zeros(128, np.float32); r[7] = np.float32(2.0 ** -24); rows.append(r)
    else:
        r = base * np.float32(2.0 ** -130); rows.append(r)        # fp32 subnormals
        r = base / np.abs(base).max() * np.float32(3.3e38); rows.append(r)
        r = base * np.float32(2.0 ** -90); rows.append(r)
    x = np.stack(rows).astype(np.float32)
    if kind == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    if kind == "fp16":
        return f16_bits_to_f32(f32_to_f16_bits(x))
    return x
