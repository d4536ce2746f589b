"""Pins the oracle's hyper-connection read (src/hc.cuh k_hc; orc_hc_read) against a float64 restatement from its
definition (tests/hc_util.py): the fold of the last half's output into R, the slices' square sums and partial dots,
inject, and mixed and its q8_1."""
import numpy as np
import pytest

from tests.hc_util import hc_inputs, hc_read_f64


def weights(orc, w):
    return orc.HcWeights(w["N"], w["HC"], w["LR"], w["w_norm"], w["dq"], w["dd"], w["uq"], w["ud"], w["w_inj"])


@pytest.mark.parametrize("N,HC,LR,fold", [(512, 4, 64, True), (1024, 4, 320, False), (512, 2, 96, True)])
def test_hc_read_against_float64(orc, N, HC, LR, fold):
    T = 3
    w, R, bo, inj = hc_inputs(N, HC, LR, T, 5 + N + LR)
    mixed, inject, xq, Rp, part, ssp = orc.hc_read(weights(orc, w), R, bo if fold else None, inj if fold else None)
    m64, i64, R64, p64, s64 = hc_read_f64(w, R, bo if fold else None, inj)
    # R' and the square sums: fp32 rounding of the float64 values
    assert np.allclose(Rp, R64, rtol=1e-6, atol=1e-6)
    if not fold:
        assert np.array_equal(Rp, R)
    assert np.allclose(ssp, s64, rtol=1e-5)
    # the partial dots (int8 dots of the same quantized xs): fp32 rounding only
    scale = np.abs(p64).max()
    assert np.abs(part - p64).max() <= 1e-5 * scale
    # inject and mixed: through silu / sigmoid and lo's int8 rounding (a q may move by one where the two land on a
    # rounding boundary)
    assert np.abs(inject - i64).max() <= 1e-4 * np.abs(i64).max()
    assert np.abs(mixed - m64).max() <= 2e-3 * np.abs(m64).max()
    # xq is mixed as q8_1
    assert np.array_equal(xq, orc.quantize_q8_1(mixed).reshape(-1))


def test_hc_read_without_inject_rows(orc):
    """w_inj null (the head's read, src/engine.cu:1049): inject untouched, the rest as with it"""
    w, R, bo, inj = hc_inputs(512, 4, 64, 2, 9)
    m1, i1, _, _, p1, _ = orc.hc_read(weights(orc, w), R, bo, inj)
    w2 = dict(w, w_inj=None)
    m2, i2, _, _, p2, _ = orc.hc_read(weights(orc, w2), R, bo, inj)
    assert np.array_equal(m1, m2) and np.array_equal(p1[:, :, :64], p2[:, :, :64])
    assert (i2 == 0).all() and (p2[:, :, 64:] == 0).all()


def test_hc_read_zero_stream_block(orc):
    """a 32-block of xs that is all zero quantizes to d = 0, q = 0 (no division by zero)"""
    w, R, bo, inj = hc_inputs(512, 4, 64, 1, 11)
    R[0, :32] = 0.0
    mixed, *_ = orc.hc_read(weights(orc, w), R)
    assert np.isfinite(mixed).all()
