"""Writes the golden fixtures of tests/golden/ from the REFERENCE ITSELF.

Runs only where oracle/_ref/libinferop_ref.so exists, i.e. where oracle/Makefile
could compile the reference's reference/reference.cpp and fp8.h from
/root/reference.  The fixtures are data (inputs and the reference's outputs);
no reference source is copied.

  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
import datagen  # noqa: E402


def encode_checksum_ref() -> int:
    R = oracle.ref()
    total = np.uint64(0)
    chunk = 1 << 26
    for lo in range(0, 1 << 32, chunk):
        out = np.empty(chunk, np.uint8)
        R.ref_encode_range(lo, lo + chunk, oracle._ptr(out, oracle._u8p))
        i = np.arange(lo, lo + chunk, dtype=np.uint64)
        w = (i * np.uint64(2654435761)) & np.uint64(0xFFFFFFFF)
        total = total + np.sum(out.astype(np.uint64) * w, dtype=np.uint64)
    return int(total)


def main() -> None:
    assert oracle.ref_available(), "oracle/_ref not built: run make -C oracle"
    R = oracle.ref()

    # M=16, N=512, K=1024, seed 0, bf16 A, bf16 out
    m, n, k = 16, 512, 1024
    a_bits, a_f32, bq, bs = datagen.gemm_case(m, n, k, seed=0)
    aq, as_ = oracle.ref_quant(a_f32)
    c = oracle.ref_gemm(aq, as_, bq, bs)
    np.savez_compressed(os.path.join(HERE, "config0.npz"), a_bits=a_bits, a_q=aq, a_s=as_,
                        b_q=bq, b_s=bs, c_ref=c)

    # quantizer edge groups, per input dtype
    edges = {}
    for kind in ("bf16", "fp16", "fp32"):
        x = datagen.special_groups(kind)
        q, s = oracle.ref_quant(x)
        edges[f"{kind}_x"] = x
        edges[f"{kind}_q"] = q
        edges[f"{kind}_s"] = s
    np.savez_compressed(os.path.join(HERE, "quant_edges.npz"), **edges)

    # codec: decode of all bytes, the reference test's edge list, 2^32 checksum
    decode = [int(np.float32(R.ref_e4m3_to_float(b)).view(np.uint32)) for b in range(256)]
    edge_vals = [0.0, 1.0, 448.0, 449.0, 464.0, 479.99998, 480.0, 512.0, 1e6, 5.9604645e-8,
                 2.9802322e-8, 1.5258789e-05, 0.0146484375, 0.015624999, 0.015625, 0.0001, 1e-9,
                 1e38]
    edge = []
    for v in edge_vals:
        for sv in (v, -v):
            f = np.float32(sv)
            edge.append([int(f.view(np.uint32)), int(R.ref_float_to_e4m3(float(f)))])
    codec = {"decode_bits": decode, "encode_edges": edge,
             "encode_checksum": encode_checksum_ref(),
             "checksum_formula": "sum_i code(i) * ((i * 2654435761) mod 2^32) mod 2^64"}
    with open(os.path.join(HERE, "codec.json"), "w") as f:
        json.dump(codec, f, indent=1)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
