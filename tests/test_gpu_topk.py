"""MoE routing (reference ops.h:102-110) against the oracle restatement of
reference/reference.cpp:152-181, for the reference test's shapes
(tests/test_topk.cpp:70-74), ties and renormalize on and off.

The device evaluates exp correctly rounded (double precision, one rounding);
the host's expf, which the reference and the oracle call, is within 0.502 ulp
and rounds the other way in about 6 of 10^4 of these inputs.  The expert ids
must therefore be identical (an id can only move if a misrounded exp breaks an
exact tie, which the tie tests below exercise with exactly representable
probabilities), and each weight within 4 ulps of the oracle's (the sum l and
the renormalizing sum inherit the last-bit differences); on inputs whose
exponentials both sides round alike the weights are bit-exact."""
import numpy as np
import pytest
import torch

import inferop_amd as ia
import oracle
from gpu_util import device, to_dev

pytestmark = pytest.mark.gpu


def _gpu(lg: np.ndarray, k: int, renorm: bool):
    t, e = lg.shape
    ids = torch.full((t, k), -7, dtype=torch.int32, device="cuda:0")
    w = torch.full((t, k), -1.0, dtype=torch.float32, device="cuda:0")
    st = ia.topk_softmax(ids, w, to_dev(lg), t, e, k, renorm)
    assert st == 0, st
    torch.cuda.synchronize()
    return ids.cpu().numpy(), w.cpu().numpy()


@pytest.mark.parametrize("shape", [(257, 256, 8), (3, 8, 2), (17, 1024, 16), (4096, 256, 8),
                                   (5, 100, 100), (64, 512, 1), (33, 65, 7)])
@pytest.mark.parametrize("renorm", [True, False])
def test_topk_parity(shape, renorm):
    device()
    t, e, k = shape
    g = np.random.default_rng(t * 1000 + e)
    lg = (2.0 * g.standard_normal((t, e))).astype(np.float32)
    ids, w = _gpu(lg, k, renorm)
    ids_r, w_r = oracle.topk_softmax(lg, k, renorm)
    assert np.array_equal(ids, ids_r)
    assert np.allclose(w, w_r, rtol=4 * 2.0 ** -24, atol=0)
    exact = (w.view(np.uint32) == w_r.view(np.uint32)).mean()
    assert exact >= 0.9, exact


def test_topk_ties_and_underflow():
    device()
    g = np.random.default_rng(52)
    lg = np.zeros((6, 64), np.float32)
    lg[1, 10] = lg[1, 20] = 1.0
    lg[2] = np.round(g.standard_normal(64))
    lg[3, :] = -120.0
    lg[3, 5] = 0.0
    lg[4, ::2] = 3.0
    lg[5] = np.float32(1e-7) * np.arange(64, dtype=np.float32)
    for renorm in (True, False):
        ids, w = _gpu(lg, 6, renorm)
        ids_r, w_r = oracle.topk_softmax(lg, 6, renorm)
        assert np.array_equal(ids, ids_r)
        assert np.array_equal(w.view(np.uint32), w_r.view(np.uint32))


def test_topk_ties_across_lanes_and_slots():
    """256 experts (four per lane): equal maxima held by one lane, by several
    lanes, and by several slots of one lane, so both ways the kernel picks
    the lowest expert among equal probabilities are taken."""
    device()
    g = np.random.default_rng(77)
    lg = np.round(g.standard_normal((40, 256))).astype(np.float32)  # many ties
    lg[0] = 0.0                                   # every expert tied
    lg[1] = -5.0
    lg[1, [5, 69, 133, 197]] = 2.0                # one lane (5), all four slots
    lg[2] = -5.0
    lg[2, [200, 7, 130, 63]] = 2.0                # four lanes, different slots
    lg[3] = -5.0
    lg[3, 250] = 3.0                              # one holder, then a tie
    lg[3, [64, 1]] = 2.0
    for k, renorm in ((8, True), (8, False), (13, True)):
        ids, w = _gpu(lg, k, renorm)
        ids_r, w_r = oracle.topk_softmax(lg, k, renorm)
        assert np.array_equal(ids, ids_r)
        assert np.allclose(w, w_r, rtol=4 * 2.0 ** -24, atol=0)
    assert list(ids_r[1, :4]) == [5, 69, 133, 197] and list(ids_r[2, :4]) == [7, 63, 130, 200]


def test_topk_rejected_calls():
    device()
    S = ia.Status
    ids = torch.full((4, 2), -7, dtype=torch.int32, device="cuda:0")
    w = torch.full((4, 2), -1.0, dtype=torch.float32, device="cuda:0")
    lg = torch.zeros((4, 8), dtype=torch.float32, device="cuda:0")
    f = ia.topk_softmax
    assert f(ids, w, lg, 0, 8, 2) == S.ERR_SHAPE
    assert f(ids, w, lg, 4, 0, 2) == S.ERR_SHAPE
    assert f(ids, w, lg, 4, 1025, 2) == S.ERR_SHAPE
    assert f(ids, w, lg, 4, 8, 0) == S.ERR_SHAPE
    assert f(ids, w, lg, 4, 8, 9) == S.ERR_SHAPE
    torch.cuda.synchronize()
    assert (ids == -7).all() and (w == -1.0).all()
