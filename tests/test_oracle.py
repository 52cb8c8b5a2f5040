"""The CPU oracle pinned against the compiled reference, an independent
encoder, closed forms and the reference tests' own known answers."""
import math

import numpy as np
import pytest

import datagen
import oracle

needs_ref = pytest.mark.skipif(not oracle.ref_available(),
                               reason="oracle/_ref not built (reference sources absent)")


def _grid_value(b: int) -> float:
    """OCP E4M3FN closed form (tests/test_fp8.cpp:8-24 describes the same)."""
    sign = -1.0 if b & 0x80 else 1.0
    e, m = (b >> 3) & 0xF, b & 7
    if e == 15 and m == 7:
        return math.nan
    if e == 0:
        return sign * m * 2.0 ** -9
    return sign * (1 + m / 8) * 2.0 ** (e - 7)


def test_decode_all_bytes_closed_form():
    L = oracle.lib()
    for b in range(256):
        want = _grid_value(b)
        got = L.orc_e4m3_to_float(b)
        if math.isnan(want):
            assert math.isnan(got)
        else:
            assert got == want and math.copysign(1, got) == (-1 if b & 0x80 else 1)


def test_encode_reference_edge_list():
    # tests/test_fp8.cpp:75-80 edge magnitudes, both signs, against the
    # independent grid encoder
    L = oracle.lib()
    for v in [0.0, 1.0, 448.0, 449.0, 464.0, 479.99998, 480.0, 512.0, 1e6, 5.9604645e-8,
              2.9802322e-8, 1.5258789e-05, 0.0146484375, 0.015624999, 0.015625, 0.0001, 1e-9, 1e38]:
        for s in (v, -v):
            assert L.orc_float_to_e4m3(s) == L.orc_grid_encode(s), s


def test_encode_grid_points_and_ties():
    # every grid point and every midpoint (tests/test_fp8.cpp:82-91)
    L = oracle.lib()
    for b in range(1, 0x7E):
        v, nxt = _grid_value(b), _grid_value(b + 1)
        assert L.orc_float_to_e4m3(v) == b
        mid = (v + nxt) / 2
        want = b if b % 2 == 0 else b + 1  # tie goes to the even encoding
        assert L.orc_float_to_e4m3(mid) == want, (b, mid)
    assert L.orc_float_to_e4m3(464.0) == 0x7E and L.orc_float_to_e4m3(-464.0) == 0xFE
    assert L.orc_float_to_e4m3(float("inf")) == 0x7E
    assert L.orc_float_to_e4m3(float("nan")) & 0x7F == 0x7F


@pytest.mark.slow
def test_encode_exhaustive_vs_independent_grid():
    assert oracle.lib().orc_sweep_encode_vs_grid(0, 1 << 32) == 0


@pytest.mark.slow
@needs_ref
def test_encode_exhaustive_vs_reference():
    L, R = oracle.lib(), oracle.ref()
    chunk = 1 << 27
    a = np.empty(chunk, np.uint8)
    b = np.empty(chunk, np.uint8)
    for lo in range(0, 1 << 32, chunk):
        L.orc_encode_range(lo, lo + chunk, oracle._ptr(a, oracle._u8p))
        R.ref_encode_range(lo, lo + chunk, oracle._ptr(b, oracle._u8p))
        assert np.array_equal(a, b), hex(lo)


@pytest.mark.slow
@needs_ref
@pytest.mark.parametrize("kind", ["bf16", "half"])
def test_16bit_conversions_exhaustive_vs_reference(kind):
    L, R = oracle.lib(), oracle.ref()
    fo = getattr(L, f"orc_{kind}_range")
    fr = getattr(R, f"ref_{kind}_range")
    chunk = 1 << 27
    a = np.empty(chunk, np.uint16)
    b = np.empty(chunk, np.uint16)
    for lo in range(0, 1 << 32, chunk):
        fo(lo, lo + chunk, oracle._ptr(a, oracle._u16p))
        fr(lo, lo + chunk, oracle._ptr(b, oracle._u16p))
        assert np.array_equal(a, b), hex(lo)


def test_half_to_float_all_vs_numpy():
    L = oracle.lib()
    h = np.arange(65536, dtype=np.uint32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([L.orc_half_to_float(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float_to_half_matches_ieee_outside_documented_departures():
    # common.h:80-101 is IEEE RNE except (65504, 65520) -> Inf and (2^-25, 2^-24) -> 0
    L = oracle.lib()
    g = np.random.default_rng(5)
    x = np.concatenate([g.standard_normal(20000).astype(np.float32) * s
                        for s in (1e-6, 1e-3, 1.0, 1e3, 3e4)])
    for v in x:
        a = abs(float(v))
        if 65504 < a < 65520 or 2.0 ** -25 < a < 2.0 ** -24:
            continue
        with np.errstate(over="ignore"):
            want = int(np.float16(v).view(np.uint16))
        assert L.orc_float_to_half(float(v)) == want, v


@needs_ref
@pytest.mark.parametrize("dist", ["normal", "stress"])
@pytest.mark.parametrize("shape", [(16, 1024), (64, 768), (77, 7168)])
def test_quant_matches_reference(shape, dist):
    m, k = shape
    x = datagen.bf16_bits_to_f32(datagen.f32_to_bf16_bits(datagen.activations(m, k, 7, dist)))
    q, s = oracle.quant(x)
    qr, sr = oracle.ref_quant(x)
    assert np.array_equal(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("kind", ["bf16", "fp16", "fp32"])
def test_quant_edge_groups_match_reference(kind):
    x = datagen.special_groups(kind)
    q, s = oracle.quant(x)
    qr, sr = oracle.ref_quant(x)
    assert np.array_equal(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))


def test_quant_zero_group_known_answer():
    # tests/test_quant.cpp:34-41: zero group -> scale exactly 1, all bytes 0
    q, s = oracle.quant(np.zeros((1, 768), np.float32))
    assert (s == 1.0).all() and (q == 0).all()


def test_quant_scale_closed_form_and_roundtrip_bound():
    # scale = absmax * fl32(1/448); round trip within the E4M3 grid bound
    # (tests/test_quant.cpp:23-32)
    x = datagen.activations(64, 768, 11)
    q, s = oracle.quant(x)
    amax = np.abs(x.reshape(64, 6, 128)).max(-1)
    inv448 = np.float32(1.0) / np.float32(448.0)
    assert np.float32(inv448).view(np.uint32) == 0x3B124925
    assert np.array_equal(s, (amax * inv448).astype(np.float32))
    dq = oracle.dequant(q, s)
    sg = np.repeat(s, 128, axis=1)
    tol = np.maximum(np.abs(x) / 16, sg * 1.5e-3) + 1e-30
    assert (np.abs(dq - x) <= tol).all()
    # the group maximum always lands on +-448
    idx = np.abs(x.reshape(64, 6, 128)).argmax(-1)
    qg = q.reshape(64, 6, 128)
    assert (np.take_along_axis(qg, idx[..., None], -1) & 0x7F == 0x7E).all()


def _dequant_f64(q, s, n_block=False):
    table = oracle.e4m3_decode_table().astype(np.float64)
    v = table[q]
    if n_block:
        sb = np.repeat(np.repeat(s, 128, axis=0)[:q.shape[0]], 128, axis=1)
    else:
        sb = np.repeat(s, 128, axis=1)
    return v * sb.astype(np.float64)


@needs_ref
def test_gemm_bit_exact_vs_reference():
    a_bits, a_f32, bq, bs = datagen.gemm_case(33, 300, 512, seed=3)
    aq, as_ = oracle.quant(a_f32)
    c = oracle.gemm(aq, as_, bq, bs)
    cr = oracle.ref_gemm(aq, as_, bq, bs)
    assert np.array_equal(c.view(np.uint32), cr.view(np.uint32))
    rows = np.array([0, 5, 32])
    assert np.array_equal(oracle.gemm_rows(aq, as_, bq, bs, rows), c[rows])


def test_gemm_thread_count_does_not_change_bits():
    # the oracle splits the output into (row, 64-column block) items across
    # threads; each element keeps the reference's summation order
    a_bits, a_f32, bq, bs = datagen.gemm_case(3, 200, 256, seed=8)
    aq, as_ = oracle.quant(a_f32)
    one = oracle.gemm(aq, as_, bq, bs, threads=1)
    assert np.array_equal(one.view(np.uint32), oracle.ref_gemm(aq, as_, bq, bs).view(np.uint32))
    for t in (2, 5, 8):
        assert np.array_equal(oracle.gemm(aq, as_, bq, bs, threads=t).view(np.uint32),
                              one.view(np.uint32))
    rows = np.array([2, 0])
    assert np.array_equal(oracle.gemm_rows(aq, as_, bq, bs, rows, threads=3), one[rows])


def test_gemm_vs_float64_matmul_of_dequantized_operands():
    a_bits, a_f32, bq, bs = datagen.gemm_case(20, 260, 384, seed=4)
    aq, as_ = oracle.quant(a_f32)
    c = oracle.gemm(aq, as_, bq, bs)
    # products of fp32-rounded dequantized values, summed in fp64: the oracle's
    # own definition; here computed by numpy's matmul
    da = (oracle.e4m3_decode_table()[aq] * np.repeat(as_, 128, axis=1)).astype(np.float64)
    sb = np.repeat(np.repeat(bs, 128, axis=0)[:260], 128, axis=1)
    db = (oracle.e4m3_decode_table()[bq] * sb).astype(np.float64)
    want = da @ db.T
    assert np.allclose(c, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())


def test_gemm_linear_in_scales_and_k_permutation_invariant():
    a_bits, a_f32, bq, bs = datagen.gemm_case(8, 130, 256, seed=6)
    aq, as_ = oracle.quant(a_f32)
    c = oracle.gemm(aq, as_, bq, bs).astype(np.float64)
    # doubling every activation scale doubles C exactly (power-of-two scaling)
    c2 = oracle.gemm(aq, as_ * 2, bq, bs).astype(np.float64)
    assert np.array_equal(c2, 2 * c)
    # zeroing the scales of group 1 removes exactly that group's contribution
    as0 = as_.copy()
    as0[:, 1] = 0
    c_g0 = oracle.gemm(aq, as0, bq, bs).astype(np.float64)
    as1 = as_.copy()
    as1[:, 0] = 0
    c_g1 = oracle.gemm(aq, as1, bq, bs).astype(np.float64)
    # each side is one fp64 sum rounded once to fp32 (<= 2^-24 relative)
    bound = 2.0 ** -23 * (np.abs(c_g0) + np.abs(c_g1) + np.abs(c))
    assert (np.abs(c_g0 + c_g1 - c) <= bound).all()
    # permuting K inside a group (same permutation on A and B) leaves C unchanged
    perm = np.random.default_rng(0).permutation(128)
    cols = np.concatenate([perm, 128 + np.arange(128)])
    cp = oracle.gemm(aq[:, cols], as_, bq[:, cols], bs).astype(np.float64)
    assert np.allclose(cp, c, rtol=0, atol=1e-6 * np.abs(c).max())


def test_weight_block_quant_properties():
    w = datagen.weights(200, 256, 9, "stress")
    bq, bs = oracle.weight_block_quant(w)
    assert bs.shape == (2, 2)
    for nb in range(2):
        for g in range(2):
            blk = w[nb * 128:(nb + 1) * 128, g * 128:(g + 1) * 128]
            amax = np.abs(blk).max()
            assert bs[nb, g] == np.float32(amax * (np.float32(1) / np.float32(448)))
            qb = bq[nb * 128:(nb + 1) * 128, g * 128:(g + 1) * 128]
            # the block maximum encodes to +-448
            i = np.unravel_index(np.abs(blk).argmax(), blk.shape)
            assert qb[i] & 0x7F == 0x7E
            deq = oracle.e4m3_decode_table()[qb] * bs[nb, g]
            assert (np.abs(deq - blk) <= np.maximum(np.abs(blk) / 16, bs[nb, g] * 1.5e-3) + 1e-30).all()


def _find_mul_div_splits(count: int, seed: int = 7):
    """(absmax, x) pairs where e4m3(fl(x * fl(1/s))) != e4m3(fl(x / s)) for the
    block scale s = fl(absmax * fl(1/448)): values sitting at an E4M3 rounding
    midpoint, where the reciprocal product and the quotient round apart."""
    g = np.random.default_rng(seed)
    L = oracle.lib()
    mids = [1.0625, 1.1875, 1.3125, 1.4375, 2.125, 2.375, 3.25, 5.5, 9.0, 13.0, 0.53125]
    out = []
    inv448 = np.float32(1) / np.float32(448)
    while len(out) < count:
        amax = np.float32(g.uniform(0.01, 10.0))
        s = np.float32(amax * inv448)
        inv = np.float32(np.float32(1) / s)
        for t in mids:
            for d in (-1, 0, 1):
                x = np.nextafter(np.float32(t * s), np.float32(np.inf if d > 0 else -np.inf)) \
                    if d else np.float32(t * s)
                if abs(x) > amax:
                    continue
                cm = L.orc_grid_encode(float(np.float32(x * inv)))
                cd = L.orc_grid_encode(float(np.float32(x / s)))
                if cm != cd:
                    out.append((amax, np.float32(x)))
    return out[:count]


def test_weight_block_quant_multiplies_by_reciprocal():
    # tests/test_gemm.cpp:38-42: w * (1 / scale), not w / scale.  Every block
    # holds its absmax plus values for which the two round to different E4M3
    # codes; the expected bytes come from numpy float32 products and the
    # independent grid encoder.
    pairs = _find_mul_div_splits(24)
    L = oracle.lib()
    w = np.zeros((128, 128 * len(pairs)), np.float32)
    for b, (amax, x) in enumerate(pairs):
        w[0, b * 128] = amax
        w[1:, b * 128 + 1] = x
        w[5, b * 128 + 7] = -x
    bq, bs = oracle.weight_block_quant(w)
    inv448 = np.float32(1) / np.float32(448)
    differ = 0
    for b, (amax, x) in enumerate(pairs):
        s = np.float32(amax * inv448)
        assert bs[0, b] == s
        inv = np.float32(np.float32(1) / s)
        for v, (r, c) in ((x, (1, b * 128 + 1)), (-x, (5, b * 128 + 7)), (amax, (0, b * 128))):
            assert bq[r, c] == L.orc_grid_encode(float(np.float32(v * inv))), (amax, v)
            differ += bq[r, c] != L.orc_grid_encode(float(np.float32(v / s)))
    assert differ >= len(pairs)


@pytest.mark.skipif(not oracle.ref_available(), reason="reference build not present")
def test_producers_bit_exact_vs_reference():
    # reference.cpp:11-35, 55-64 compiled from the reference sources
    import ctypes
    R = oracle.ref()
    g = np.random.default_rng(21)
    gu = (3.0 * g.standard_normal((33, 2 * 384))).astype(np.float32)
    gu[0, :8] = [0.0, -0.0, 88.0, -88.0, 100.0, -104.0, 1e-30, -1e-30]
    want = np.empty((33, 384), np.float32)
    R.ref_silu_and_mul(want.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                       gu.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 33, 384)
    got = oracle.silu_and_mul(gu)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    res = g.standard_normal((17, 1536)).astype(np.float32)
    x = g.standard_normal((17, 1536)).astype(np.float32)
    w = (1.0 + 0.1 * g.standard_normal(1536)).astype(np.float32)
    r2, out = oracle.fused_add_rmsnorm(res, x, w, 1e-6)
    rr = res.copy()
    out_ref = np.empty_like(res)
    fp = ctypes.POINTER(ctypes.c_float)
    R.ref_fused_add_rmsnorm(rr.ctypes.data_as(fp), out_ref.ctypes.data_as(fp),
                            x.ctypes.data_as(fp), w.ctypes.data_as(fp), 17, 1536, 1e-6)
    assert np.array_equal(r2.view(np.uint32), rr.view(np.uint32))
    assert np.array_equal(out.view(np.uint32), out_ref.view(np.uint32))
    y = oracle.rmsnorm(x, w, 1e-5)
    y_ref = np.empty_like(x)
    R.ref_rmsnorm(y_ref.ctypes.data_as(fp), x.ctypes.data_as(fp), w.ctypes.data_as(fp), 17, 1536,
                  1e-5)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))


def test_producers_closed_forms():
    # SiLU within a few fp32 ulps of the float64 formula; RMSNorm exact on
    # integer inputs (every product and partial sum is exact in fp32)
    g = np.random.default_rng(22)
    gu = (4.0 * g.standard_normal((8, 2 * 256))).astype(np.float32)
    got = oracle.silu_and_mul(gu).astype(np.float64)
    gg, uu = gu[:, :256].astype(np.float64), gu[:, 256:].astype(np.float64)
    want = gg / (1.0 + np.exp(-gg)) * uu
    assert (np.abs(got - want) <= 4 * np.spacing(np.abs(want).astype(np.float32)) + 1e-37).all()
    res = g.integers(-8, 9, (4, 1024)).astype(np.float32)
    x = g.integers(-8, 9, (4, 1024)).astype(np.float32)
    w = g.integers(1, 4, 1024).astype(np.float32)
    r2, out = oracle.fused_add_rmsnorm(res, x, w, 0.0)
    assert np.array_equal(r2, res + x)
    ss = (r2.astype(np.float64) ** 2).sum(axis=1, keepdims=True)
    inv = np.float32(1) / np.sqrt((ss / 1024).astype(np.float32)).astype(np.float32)
    assert np.array_equal(out, (r2 * inv) * w)


def _topk_cases():
    g = np.random.default_rng(51)
    yield (2.0 * g.standard_normal((257, 256))).astype(np.float32), 8
    yield (2.0 * g.standard_normal((3, 8))).astype(np.float32), 2
    yield (2.0 * g.standard_normal((17, 1024))).astype(np.float32), 16
    tie = np.zeros((4, 64), np.float32)          # all equal: index order
    tie[1, 10] = tie[1, 20] = 1.0                # equal maxima
    tie[2] = np.round(g.standard_normal(64))     # many exact ties
    tie[3, :] = -120.0                           # probabilities that underflow together
    tie[3, 5] = 0.0
    yield tie, 6


@pytest.mark.skipif(not oracle.ref_available(), reason="reference build not present")
def test_topk_softmax_bit_exact_vs_reference():
    import ctypes
    R = oracle.ref()
    for lg, k in _topk_cases():
        for renorm in (True, False):
            ids, w = oracle.topk_softmax(lg, k, renorm)
            t, e = lg.shape
            ids_r = np.empty((t, k), np.int32)
            w_r = np.empty((t, k), np.float32)
            R.ref_topk_softmax(ids_r.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                               w_r.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                               np.ascontiguousarray(lg).ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                               t, e, k, int(renorm))
            assert np.array_equal(ids, ids_r)
            assert np.array_equal(w.view(np.uint32), w_r.view(np.uint32))


def test_topk_softmax_closed_form():
    # tests/test_topk.cpp:13-34 properties, and the float64 softmax order
    for lg, k in _topk_cases():
        ids, w = oracle.topk_softmax(lg, k, True)
        assert np.allclose(w.sum(axis=1), 1.0, atol=1e-5)
        assert (np.diff(w, axis=1) <= 0).all()
        assert all(len(set(r)) == k for r in ids)
        p = np.exp(lg.astype(np.float64) - lg.max(axis=1, keepdims=True))
        for r in range(lg.shape[0]):
            # float64 order with index tie-break agrees wherever fp32 keeps values apart
            o = sorted(range(lg.shape[1]), key=lambda e: (-p[r, e], e))[:k]
            pf = np.float32(p[r])
            if len(set(pf[o].tolist())) == k and len(np.unique(pf)) == lg.shape[1]:
                assert list(ids[r]) == o
        _, w0 = oracle.topk_softmax(lg, k, False)
        l = np.exp(lg.astype(np.float64) - lg.max(axis=1, keepdims=True)).sum(axis=1, keepdims=True)
        assert np.allclose(w0, np.sort(p / l, axis=1)[:, ::-1][:, :k], rtol=1e-5, atol=1e-9)


def _dequant_cases(gs):
    """(q, s) pairs: seeded quantizer outputs of normal and stress activations,
    every byte value (NaN codes 0x7F/0xFF included) under scales spanning the
    fp32 range (subnormal, 1, huge enough to overflow), and the quantizer's
    edge groups (zeros, Inf/NaN, denormal inputs)."""
    out = []
    for dist in ("normal", "stress"):
        x = datagen.activations(24, 10 * gs, 31 + gs, dist)
        out.append(oracle.quant(x, gs))
    g = np.random.default_rng(gs)
    q = np.tile(np.arange(256, dtype=np.uint8), (6, (2 * gs + 255) // 256))[:, :2 * gs]
    q = np.ascontiguousarray(np.concatenate([q, g.integers(0, 256, (6, 2 * gs), dtype=np.uint8)],
                                            axis=1))
    s = np.array([[1.0, 2.0 ** -149, 3.5e-39, 0.0123, 1e30, 3.4e38, 7.0, -0.5][i % 8]
                  for i in range(6 * 4)], np.float32).reshape(6, 4)
    out.append((q, s))
    if gs == 128:
        for kind in ("bf16", "fp16", "fp32"):
            out.append(oracle.quant(datagen.special_groups(kind)))
    return out


@needs_ref
@pytest.mark.parametrize("gs", [128, 64, 48, 40])
def test_dequant_matches_reference(gs):
    # reference.cpp:82-91: x = e4m3_to_float(q) * scale, an fp32 product
    for q, s in _dequant_cases(gs):
        got = oracle.dequant(q, s, gs)
        want = oracle.ref_dequant(q, s, gs)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("gs", [128, 64, 48, 40])
def test_dequant_closed_form(gs):
    # the same cases against the closed form: the E4M3 value (the 256-entry
    # table pinned by the OCP definition) times its group's scale, rounded to
    # fp32 by numpy; NaN codes give NaN (compared as NaN)
    table = oracle.e4m3_decode_table()
    for q, s in _dequant_cases(gs):
        with np.errstate(over="ignore", invalid="ignore"):
            want = table[q] * np.repeat(s, gs, axis=1)
        got = oracle.dequant(q, s, gs)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_silu_bf16_exponent_rules():
    # The bf16 SiLU kernel keeps only gates with exponent field in [102, 134)
    # in its LDS table and computes the rest as g * 0.5 (E < 102), g (E >= 134,
    # g > 0; also +Inf and positive NaN) or -0 (E >= 134 finite, g < 0); -Inf
    # and negative NaN read the full table.  Check every bf16 pattern against
    # the oracle's SiLU (reference.cpp:55-64 with up = 1).
    bits = np.arange(65536, dtype=np.uint32)
    gate = (bits << 16).view(np.float32)
    gu = np.concatenate([gate.reshape(-1, 128), np.ones((512, 128), np.float32)], axis=1)
    with np.errstate(all="ignore"):
        want = oracle.silu_and_mul(gu).reshape(-1)
        e = (bits >> 7) & 0xFF
        neg = (bits >> 15) == 1
        rule = np.where(e < 102, gate * np.float32(0.5),
                        np.where(neg, np.float32(-0.0), gate)).astype(np.float32)
    outside = (e < 102) | ((e >= 134) & ~(neg & (e == 255)))
    got, exp = rule[outside], want[outside]
    same = (got.view(np.uint32) == exp.view(np.uint32)) | (np.isnan(got) & np.isnan(exp))
    assert same.all(), bits[outside][~same][:8]
    assert (np.signbit(got) == np.signbit(exp)).all()
    # the rules are not vacuous: inside the table range they fail somewhere
    inside = (e >= 102) & (e < 134)
    assert (rule[inside].view(np.uint32) != want[inside].view(np.uint32)).sum() > 1000
