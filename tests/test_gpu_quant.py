"""GPU quantizer / dequantizer parity with the oracle: bytes and scales
bit-exact (reference/reference.cpp:65-91 semantics on identical inputs)."""
import os

import numpy as np
import pytest
import torch

import datagen
import inferop_amd
import oracle
from gpu_util import bf16_dev, device, f16_dev, to_dev, to_np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DT = inferop_amd.dtype


def _pack(x32: np.ndarray, kind: str):
    """(device tensor, exact fp32 values the oracle must see)."""
    if kind == "bf16":
        bits = datagen.f32_to_bf16_bits(x32)
        return bf16_dev(bits), datagen.bf16_bits_to_f32(bits)
    if kind == "fp16":
        bits = datagen.f32_to_f16_bits(x32)
        return f16_dev(bits), datagen.f16_bits_to_f32(bits)
    return to_dev(x32.astype(np.float32)), x32.astype(np.float32)


def _gpu_quant(xd, kind, rows, cols, gs=128):
    q = torch.full((rows, cols), 0xA5, dtype=torch.uint8, device="cuda:0")
    s = torch.full((rows, cols // gs), -7.0, dtype=torch.float32, device="cuda:0")
    st = inferop_amd.quant_fp8_per_token_group(q, s, xd, getattr(DT, kind), rows, cols, gs)
    assert st == 0
    return to_np(q), to_np(s)


def _assert_same(q, s, qr, sr, what):
    if not np.array_equal(q, qr):
        i = np.argwhere(q != qr)[0]
        raise AssertionError(f"{what}: {int((q != qr).sum())} byte mismatches, first at {i}: "
                             f"got {q[tuple(i)]:#x} want {qr[tuple(i)]:#x}")
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32)), what


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("shape,dist", [((16, 1024), "normal"), ((1, 2048), "normal"),
                                        ((64, 7168), "normal"), ((77, 7168), "stress"),
                                        ((1000, 7168), "stress"), ((3, 128), "normal"),
                                        ((64, 768), "normal")])  # tests/test_quant.cpp:11-13
def test_quant_parity(kind, shape, dist):
    device()
    m, k = shape
    print(f"quant parity {kind} {shape} {dist}", flush=True)
    xd, x32 = _pack(datagen.activations(m, k, 21, dist), kind)
    q, s = _gpu_quant(xd, kind, m, k)
    qr, sr = oracle.quant(x32)
    _assert_same(q, s, qr, sr, f"{kind} {shape}")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["bf16", "fp16", "fp32"])
def test_quant_edge_groups_vs_reference_fixture(kind):
    # NaN / Inf / -0 / zero / subnormal / tiny / huge groups; expected bytes
    # written by the reference's own compiled code
    device()
    g = np.load(os.path.join(GOLDEN, "quant_edges.npz"))
    x = g[f"{kind}_x"]
    xd, _ = _pack(x, kind)
    q, s = _gpu_quant(xd, kind, x.shape[0], x.shape[1])
    _assert_same(q, s, g[f"{kind}_q"], g[f"{kind}_s"], f"edges {kind}")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["bf16", "fp32"])
@pytest.mark.parametrize("gs", [32, 64, 256, 96])
def test_quant_other_group_sizes(kind, gs):
    device()
    m, k = 9, gs * 6
    xd, x32 = _pack(datagen.activations(m, k, 5, "stress"), kind)
    q, s = _gpu_quant(xd, kind, m, k, gs)
    qr, sr = oracle.quant(x32, gs)
    _assert_same(q, s, qr, sr, f"gs={gs}")


@pytest.mark.gpu
def test_quant_unaligned_input_uses_generic_path():
    device()
    m, k = 4, 512
    x32 = datagen.activations(m, k + 1, 8).astype(np.float32)
    bits = datagen.f32_to_bf16_bits(x32).reshape(-1)
    buf = bf16_dev(bits)
    xd = buf[1:1 + m * k]  # 2-byte offset: not 16-byte aligned
    q, s = _gpu_quant(xd, "bf16", m, k)
    qr, sr = oracle.quant(datagen.bf16_bits_to_f32(bits[1:1 + m * k]).reshape(m, k))
    _assert_same(q, s, qr, sr, "unaligned")


@pytest.mark.gpu
def test_quant_rejected_shapes_leave_outputs_untouched():
    device()
    x = torch.zeros((4, 200), dtype=torch.bfloat16, device="cuda:0")
    q = torch.full((4, 200), 0x5A, dtype=torch.uint8, device="cuda:0")
    s = torch.full((4, 2), 3.0, dtype=torch.float32, device="cuda:0")
    S = inferop_amd.Status
    assert inferop_amd.quant_fp8_per_token_group(q, s, x, DT.bf16, 4, 200, 128) == S.ERR_SHAPE
    assert inferop_amd.quant_fp8_per_token_group(q, s, x, DT.fp8_e4m3, 4, 128, 128) == S.ERR_DTYPE
    torch.cuda.synchronize()
    assert (q == 0x5A).all() and (s == 3.0).all()


@pytest.mark.gpu
def test_quant_large_whole_tensor_and_roundtrip():
    # M=4096, K=16384 (config 2's largest K): every byte and scale against the
    # oracle, and the size-independent round-trip bound on top
    device()
    m, k = 4096, 16384
    g = torch.Generator(device="cuda:0").manual_seed(3)
    x = torch.randn((m, k), generator=g, device="cuda:0").to(torch.bfloat16)
    q = torch.empty((m, k), dtype=torch.uint8, device="cuda:0")
    s = torch.empty((m, k // 128), dtype=torch.float32, device="cuda:0")
    assert inferop_amd.quant_fp8_per_token_group(q, s, x, DT.bf16, m, k) == 0
    qr, sr = oracle.quant(datagen.bf16_bits_to_f32(to_np(x).view(np.uint16)))
    _assert_same(to_np(q), to_np(s), qr, sr, "4096x16384 whole tensor")
    del qr, sr
    # dequantize on the GPU and bound the error everywhere
    xd = torch.empty((m, k), dtype=torch.float32, device="cuda:0")
    assert inferop_amd.dequant_fp8_per_token_group(xd, DT.fp32, q, s, m, k) == 0
    xf = x.float()
    sg = s.repeat_interleave(128, dim=1)
    tol = torch.maximum(xf.abs() / 16, sg * 1.5e-3)
    assert bool(((xd - xf).abs() <= tol).all())
    # 16-bit outputs at this size (201 MB of codes and outputs: the
    # cached-store band of the dequantizer) are the fp32 products rounded to
    # the output type
    for odt, code in ((torch.bfloat16, DT.bf16), (torch.float16, DT.fp16)):
        xh = torch.empty((m, k), dtype=odt, device="cuda:0")
        assert inferop_amd.dequant_fp8_per_token_group(xh, code, q, s, m, k) == 0
        assert torch.equal(xh.view(torch.int16), xd.to(odt).view(torch.int16)), str(odt)
        del xh


@pytest.mark.gpu
@pytest.mark.parametrize("kind,m,k", [("fp16", 4096, 7168), ("fp16", 8192, 18432),
                                      ("fp32", 2048, 7168), ("fp32", 8192, 18432)])
def test_quant_cache_policy_sizes_whole_tensor(kind, m, k):
    # the quantizer's cached-access band (64-256 MiB of input and codes) and
    # the sizes above it, for fp16 and fp32 inputs: every byte and scale
    # against the oracle
    device()
    print(f"quant {kind} {m}x{k}", flush=True)
    g = torch.Generator(device="cuda:0").manual_seed(m + k)
    x = torch.randn((m, k), generator=g, device="cuda:0")
    if kind == "fp16":
        x = x.half()
    q = torch.empty((m, k), dtype=torch.uint8, device="cuda:0")
    s = torch.empty((m, k // 128), dtype=torch.float32, device="cuda:0")
    assert inferop_amd.quant_fp8_per_token_group(q, s, x, getattr(DT, kind), m, k) == 0
    qr, sr = oracle.quant(x.float().cpu().numpy())
    _assert_same(to_np(q), to_np(s), qr, sr, f"{kind} {m}x{k} whole tensor")


@pytest.mark.gpu
@pytest.mark.parametrize("out", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("gs", [128, 64, 48, 40, 36])  # 36: the element-wise path
def test_dequant_parity(out, gs):
    device()
    m, k = 37, gs * 8
    x32 = datagen.activations(m, k, 12, "stress")
    qr, sr = oracle.quant(x32, gs)
    want = oracle.dequant(qr, sr, gs)
    xd = torch.empty((m, k), dtype={"fp32": torch.float32, "bf16": torch.bfloat16,
                                    "fp16": torch.float16}[out], device="cuda:0")
    assert inferop_amd.dequant_fp8_per_token_group(xd, getattr(DT, out), to_dev(qr), to_dev(sr),
                                                   m, k, gs) == 0
    got = xd.float().cpu().numpy()
    # fp32: bit-exact; 16-bit: the oracle's fp32 value rounded to nearest-even
    want_t = torch.from_numpy(want).to(xd.dtype).float().numpy()
    assert np.array_equal(got.view(np.uint32), want_t.view(np.uint32))


def _e4m3_value(b: int) -> float:
    e, m = (b >> 3) & 15, b & 7
    v = m / 8 * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
    return -v if b & 0x80 else v


def _fp16_tie_cases():
    """(e4m3 byte, fp32 scale) pairs whose exact product lies just below an
    fp16 rounding midpoint and rounds to it in fp32: rounding the fp32 product
    to fp16 (ties to even, upwards here) differs from rounding the exact
    product to fp16 once (downwards)."""
    rng = np.random.default_rng(5)
    cases = []
    for b in range(1, 0x7F):
        qv = _e4m3_value(b)
        for _ in range(200):
            e, j = int(rng.integers(-8, 12)), int(rng.integers(1024, 2048)) | 1
            mid = (2 * j + 1) * 2.0 ** (e - 11)  # between odd j and even j + 1 (x 2^(e-10))
            s0 = np.float32(mid / qv)
            hit = None
            for d in range(-3, 4):
                sc = np.float32(s0 + np.float32(d) * np.spacing(s0))
                exact = qv * float(sc)  # 4 x 24 significant bits: exact in fp64
                if np.float16(np.float32(exact)).view(np.uint16) != np.float16(exact).view(np.uint16):
                    hit = sc
                    break
            if hit is not None:
                cases.append((b, hit))
                break
    return cases


@pytest.mark.gpu
@pytest.mark.parametrize("gs", [128, 64, 48, 40, 36])
def test_dequant_fp16_rounds_through_fp32(gs):
    """fp16 output is the fp32 product rounded to fp16 (two roundings, as in
    the reference), not the exact product rounded once: every group here is
    a case where the two differ."""
    device()
    cases = _fp16_tie_cases()
    assert len(cases) > 64
    m, k = 16, gs * 8
    q = np.empty((m, k), np.uint8)
    s = np.empty((m, k // gs), np.float32)
    for r in range(m):
        for c in range(k // gs):
            b, sc = cases[(r * (k // gs) + c) % len(cases)]
            q[r, c * gs:(c + 1) * gs] = b | (0x80 if (r + c) % 2 else 0)
            s[r, c] = sc
    want = torch.from_numpy(oracle.dequant(q, s, gs)).to(torch.float16).numpy()
    once = np.array([[_e4m3_value(int(q[r, j])) * float(s[r, j // gs]) for j in range(k)]
                     for r in range(m)]).astype(np.float16)
    assert not np.any(once.view(np.uint16) == want.view(np.uint16))
    xd = torch.empty((m, k), dtype=torch.float16, device="cuda:0")
    assert inferop_amd.dequant_fp8_per_token_group(xd, DT.fp16, to_dev(q), to_dev(s), m, k,
                                                   gs) == 0
    got = xd.cpu().numpy()
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
