"""The oracle against the committed golden fixtures, which were written by the
reference's own compiled CPU code (tests/golden/make_golden.py)."""
import json
import os

import numpy as np

import datagen
import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_config0_quant_and_gemm_bit_exact():
    g = np.load(os.path.join(GOLDEN, "config0.npz"))
    a = datagen.bf16_bits_to_f32(g["a_bits"])
    q, s = oracle.quant(a)
    assert np.array_equal(q, g["a_q"])
    assert np.array_equal(s.view(np.uint32), g["a_s"].view(np.uint32))
    c = oracle.gemm(g["a_q"], g["a_s"], g["b_q"], g["b_s"])
    assert np.array_equal(c.view(np.uint32), g["c_ref"].view(np.uint32))


def test_config0_inputs_regenerate_from_seed():
    g = np.load(os.path.join(GOLDEN, "config0.npz"))
    a_bits, _, bq, bs = datagen.gemm_case(16, 512, 1024, seed=0)
    assert np.array_equal(a_bits, g["a_bits"])
    assert np.array_equal(bq, g["b_q"]) and np.array_equal(bs, g["b_s"])


def test_quant_edges_bit_exact():
    g = np.load(os.path.join(GOLDEN, "quant_edges.npz"))
    for kind in ("bf16", "fp16", "fp32"):
        q, s = oracle.quant(g[f"{kind}_x"])
        assert np.array_equal(q, g[f"{kind}_q"]), kind
        assert np.array_equal(s.view(np.uint32), g[f"{kind}_s"].view(np.uint32)), kind


def test_codec_golden():
    c = json.load(open(os.path.join(GOLDEN, "codec.json")))
    L = oracle.lib()
    for b in range(256):
        got = np.float32(L.orc_e4m3_to_float(b)).view(np.uint32)
        assert int(got) == c["decode_bits"][b], b
    for bits, code in c["encode_edges"]:
        f = float(np.uint32(bits).view(np.float32))
        assert L.orc_float_to_e4m3(f) == code, hex(bits)
    assert L.orc_encode_checksum(0, 1 << 32) == c["encode_checksum"]
