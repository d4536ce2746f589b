"""Pins the oracle's expert arithmetic: the Q4_K and Q8_0 dots against float64 products of the dequantized operands,
the SwiGLU q8_1 step against its definition, and the layer's combine against a float64 weighted sum.
"""
import numpy as np
import pytest


def q81_values(yq, n):
    """dequantized q8_1 activations d * q, float64"""
    b = yq.reshape(n // 32, 36)
    d = b[:, :2].copy().view(np.float16)[:, 0].astype(np.float64)
    return (b[:, 4:].view(np.int8).astype(np.float64) * d[:, None]).reshape(-1)


@pytest.mark.parametrize("wtype", [12, 13, 2, 7, 8])
@pytest.mark.parametrize("K", [512, 2048])
def test_dot_against_dequantized_float64(orc, wtype, K):
    rows = 24
    w = orc.synth(rows * K, 31 + K, 0.02).reshape(rows, K)
    blk = orc.quantize(wtype, w).reshape(rows, -1)
    wd = orc.dequant(wtype, blk.reshape(-1), rows, K).astype(np.float64)
    x = orc.synth(3 * K, 32, 1.0).reshape(3, K)
    yq = orc.quantize_q8_1(x).reshape(3, -1)
    for t in range(3):
        a = q81_values(yq[t], K)
        for r in range(rows):
            got = orc.dot(wtype, blk[r], yq[t], K)
            exact = float(wd[r] @ a)
            assert abs(got - exact) <= 2e-6 * float(np.abs(wd[r]) @ np.abs(a)) + 1e-9, (r, t, got, exact)


def test_q4k_dot_is_linear_in_the_min_term(orc):
    """a block whose scales are all zero leaves only -dmin m sum(q8): doubling m doubles the dot"""
    K = 512
    blk = np.zeros((2, K // 256 * 144), np.uint8)
    for r, m in ((0, 5), (1, 10)):
        for b in range(K // 256):
            o = b * 144
            blk[r, o:o + 2] = np.frombuffer(np.float16(0.0).tobytes(), np.uint8)
            blk[r, o + 2:o + 4] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
            blk[r, o + 8:o + 12] = m     # m0..m3 (low 6 bits of bytes 4-7 of the scales)
            blk[r, o + 12:o + 16] = (m & 15) << 4   # m4..m7 low nibbles
    x = orc.synth(K, 33, 1.0).reshape(1, K)
    yq = orc.quantize_q8_1(x)
    a, b = orc.dot(12, blk[0], yq, K), orc.dot(12, blk[1], yq, K)
    assert a != 0 and b == 2 * a
    sums = yq.reshape(-1, 36)[:, 4:].view(np.int8).astype(np.float64).sum(axis=1)
    d8 = yq.reshape(-1, 36)[:, :2].copy().view(np.float16)[:, 0].astype(np.float64)
    assert np.isclose(a, -0.125 * 5 * float(d8 @ sums), rtol=1e-5)


def test_swiglu_q8_1(orc):
    ff = 512
    gu = orc.synth(2 * ff, 34, 1.0)
    hq = orc.swiglu_q8_1(gu, ff)
    g, u = gu[:ff].astype(np.float64), gu[ff:].astype(np.float64)
    h = g / (1 + np.exp(-g)) * u
    q = hq.reshape(-1, 36)[:, 4:].view(np.int8).astype(np.float64)
    d = np.abs(h.reshape(-1, 32)).max(axis=1) / 127
    assert np.all(np.abs(h.reshape(-1, 32) / d[:, None] - q) <= 0.5 + 1e-3)
    d16 = hq.reshape(-1, 36)[:, :2].copy().view(np.float16)[:, 0].astype(np.float64)
    assert np.allclose(d16, d, rtol=1e-3)


def small_layer(orc, wtype=12, H=1024, E=64, K=6, ff=512, seed=40):
    W = orc.synth((E + 1) * H, seed, 0.02).reshape(E + 1, H)
    gu = orc.quantize(wtype, orc.synth((E + 1) * 2 * ff * H, seed + 1, 0.02).reshape(-1, H))
    dn = orc.quantize(wtype, orc.synth((E + 1) * H * ff, seed + 2, 0.02).reshape(-1, ff))
    return orc.LayerWeights(W, gu, dn, wtype, H, E, K, ff, True)


@pytest.mark.parametrize("wtype", [12, 13, 2, 7, 8])
def test_layer_pieces_are_consistent(orc, wtype):
    L = small_layer(orc, wtype)
    T = 3
    x = orc.synth(T * L.H, 45, 1.0).reshape(T, L.H)
    y, logits, topi, topw, gu, part = orc.layer_decode(L, x)
    # routing as the pieces compute it
    assert np.array_equal(logits, orc.router_logits(L.W, x))
    ti, tw, _ = orc.topk(logits, L.E, L.K)
    assert np.array_equal(ti, topi) and np.array_equal(tw, topw)
    # a few gate|up and down values against the dot on the pair's expert and token
    xq = orc.quantize_q8_1(x).reshape(T, -1)
    gurb = orc.row_bytes(wtype, L.H)
    dnrb = orc.row_bytes(wtype, L.ff)
    rng = np.random.default_rng(0)
    P = T * L.K
    for _ in range(40):
        p = int(rng.integers(0, P + T))
        e, t = (topi.reshape(-1)[p], p // L.K) if p < P else (L.E, p - P)
        r = int(rng.integers(0, 2 * L.ff))
        w = L.gu_w[e * L.gu_stride + r * gurb: e * L.gu_stride + (r + 1) * gurb]
        assert gu[p, r] == orc.dot(wtype, w, xq[t], L.H)
        hq = orc.swiglu_q8_1(gu[p], L.ff)
        r2 = int(rng.integers(0, L.H))
        w2 = L.dn_w[e * L.dn_stride + r2 * dnrb: e * L.dn_stride + (r2 + 1) * dnrb]
        assert part[p, r2] == orc.dot(wtype, w2, hq, L.ff)
    # the combine: the weighted sum in float64
    sig = 1 / (1 + np.exp(-logits[:, L.E].astype(np.float64)))
    want = np.einsum("tk,tkh->th", topw.astype(np.float64), part[:P].reshape(T, L.K, L.H).astype(np.float64))
    want += sig[:, None] * part[P:].astype(np.float64)
    assert np.allclose(y, want, rtol=1e-5, atol=1e-6)
    # threads change nothing
    y4 = orc.layer_decode(L, x, nthreads=4)[0]
    assert np.array_equal(y, y4)


@pytest.mark.parametrize("K", [512, 2048])
def test_q8s_dot_against_float64_and_its_lane_order(orc, K):
    """the shared expert's dense Q8_0 dot (src/dense.cuh:24-154): within fp32 rounding of the float64 product of the
    dequantized operands; and its own order, not the routed Q8_0 dot's: the two differ in the last bits on most rows
    (a restatement that fell back to the routed lanes would be caught here)"""
    rows = 32
    w = orc.quantize(orc.Q8_0, orc.synth(rows * K, 51 + K, 0.02).reshape(rows, K)).reshape(rows, -1)
    wd = orc.dequant(orc.Q8_0, w.reshape(-1), rows, K).astype(np.float64)
    yq = orc.quantize_q8_1(orc.synth(K, 52, 1.0).reshape(1, K))
    a = q81_values(yq, K)
    differ = 0
    for r in range(rows):
        got = orc.dot_q8s(w[r], yq, K)
        exact = float(wd[r] @ a)
        assert abs(got - exact) <= 2e-6 * float(np.abs(wd[r]) @ np.abs(a)) + 1e-9
        differ += got != orc.dot(orc.Q8_0, w[r], yq, K)
    assert differ >= rows // 4


def test_q8s_dot_single_half_block(orc):
    """one 16-column half in lane 0 only: the dot is exactly (d_w d_a) sum q_w q_a, rounded once"""
    K = 512
    w = np.zeros((K // 32, 34), np.uint8)
    y = np.zeros((K // 32, 36), np.uint8)
    w[:, :2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    y[:, :2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    qw = np.arange(1, 17, dtype=np.int8)
    qa = np.arange(-8, 8, dtype=np.int8)
    w[0, 2:18] = qw.view(np.uint8)        # columns 0..15: lane 0's first half
    y[0, 4:20] = qa.view(np.uint8)
    want = np.float32(0.125) * np.float32(int(qw.astype(np.int32) @ qa.astype(np.int32)))
    assert orc.dot_q8s(w.reshape(-1), y.reshape(-1), K) == want
