"""The product's host headers (include/inferop/fp8.h, common.h) and the
quantizer's quotient arithmetic, checked exhaustively on the CPU."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
HC_PATH = os.path.join(HERE, "native", "libhostcheck.so")
_hc = None


def hc():
    global _hc
    if _hc is None:
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "native")], check=True)
        L = ctypes.CDLL(HC_PATH)
        L.hc_encode_range.argtypes = [ctypes.c_uint64, ctypes.c_uint64, oracle._u8p]
        L.hc_bf16_range.argtypes = [ctypes.c_uint64, ctypes.c_uint64, oracle._u16p]
        L.hc_half_range.argtypes = [ctypes.c_uint64, ctypes.c_uint64, oracle._u16p]
        L.hc_decode.restype = ctypes.c_float
        L.hc_decode.argtypes = [ctypes.c_uint8]
        L.hc_half_to_float.restype = ctypes.c_float
        L.hc_half_to_float.argtypes = [ctypes.c_uint16]
        L.hc_bf16_to_float.restype = ctypes.c_float
        L.hc_bf16_to_float.argtypes = [ctypes.c_uint16]
        L.hc_markstein_sweep.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_uint64)]
        _hc = L
    return _hc


def test_decode_header_vs_oracle_all_bytes():
    L, O = hc(), oracle.lib()
    for b in range(256):
        a, r = L.hc_decode(b), O.orc_e4m3_to_float(b)
        assert np.float32(a).view(np.uint32) == np.float32(r).view(np.uint32) or (a != a and r != r)
        if a != a:
            assert np.signbit(np.float32(a)) == bool(b & 0x80)


@pytest.mark.slow
def test_encode_header_exhaustive_vs_oracle():
    L, O = hc(), oracle.lib()
    chunk = 1 << 27
    a = np.empty(chunk, np.uint8)
    b = np.empty(chunk, np.uint8)
    for lo in range(0, 1 << 32, chunk):
        L.hc_encode_range(lo, lo + chunk, oracle._ptr(a, oracle._u8p))
        O.orc_encode_range(lo, lo + chunk, oracle._ptr(b, oracle._u8p))
        assert np.array_equal(a, b), hex(lo)


@pytest.mark.slow
@pytest.mark.parametrize("kind", ["bf16", "half"])
def test_16bit_header_conversions_exhaustive_vs_oracle(kind):
    L, O = hc(), oracle.lib()
    fh = getattr(L, f"hc_{kind}_range")
    fo = getattr(O, f"orc_{kind}_range")
    chunk = 1 << 27
    a = np.empty(chunk, np.uint16)
    b = np.empty(chunk, np.uint16)
    for lo in range(0, 1 << 32, chunk):
        fh(lo, lo + chunk, oracle._ptr(a, oracle._u16p))
        fo(lo, lo + chunk, oracle._ptr(b, oracle._u16p))
        assert np.array_equal(a, b), hex(lo)


def test_16bit_header_decodes_all_patterns():
    L, O = hc(), oracle.lib()
    for h in range(65536):
        a, b = L.hc_half_to_float(h), O.orc_half_to_float(h)
        assert (np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)) or (a != a and b != b)
        # (ctypes returns through a Python float, which quiets signalling NaNs)
        v = L.hc_bf16_to_float(h)
        if v != v:
            assert (h & 0x7FFF) > 0x7F80
        else:
            assert np.float32(v).view(np.uint32) == (h << 16)


@pytest.mark.slow
@pytest.mark.parametrize("kind,name", [(0, "bf16"), (1, "fp16")])
def test_fast_path_quotient_exhaustive(kind, name):
    # every (x, absmax) pair the quantizer's fast path admits for 16-bit input:
    # the Markstein quotient gives the reference's E4M3 byte in all cases and
    # the exact IEEE quotient wherever |x/scale| >= 2^-11
    out = (ctypes.c_uint64 * 4)()
    hc().hc_markstein_sweep(kind, out)
    pairs, bad_q, bad_bytes, bad_big = list(out)
    assert pairs > 10 ** 9
    assert bad_bytes == 0
    assert bad_big == 0
    if name == "fp16":
        assert bad_q == 0
