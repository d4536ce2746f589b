"""Pins the oracle's number formats: f16 conversion and fma, Q4_K / Q8_0 layouts, dequantization, the quantizers and
q8_1 activations.  Each check comes from outside the oracle's own formulas: numpy's IEEE f16, exact rational
arithmetic, hand-built blocks with known values, and round-trip bounds derived from the format.
"""
from fractions import Fraction

import numpy as np
import pytest


# ------------------------------------------------------------------------------------------------ f16
def test_f16_to_f32_matches_numpy_on_every_pattern(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(np.isinf(got), np.isinf(ref))


def test_f32_to_f16_rounds_to_nearest_even_like_numpy(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 5000), rng.normal(0, 3e4, 5000),
        # exact ties between neighbouring f16 values (normal and subnormal) and the overflow edge
        (np.arange(1, 2000) * 2.0 ** -25), 1 + (np.arange(0, 3000) + 0.5) * 2.0 ** -10, [65504, 65519.99, 65520, 1e9, -65520],
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, ref)


_F16_SORTED = None


def _round_f16_exact(v: Fraction) -> int:
    """nearest f16 to an exact rational, ties to the even pattern (a search over all finite f16 values)"""
    global _F16_SORTED
    if _F16_SORTED is None:
        b = np.arange(0, 0x7C00, dtype=np.uint16)  # non-negative finite
        _F16_SORTED = (b, b.view(np.float16).astype(np.float64))
    bits, vals = _F16_SORTED
    neg = v < 0
    a = -v if neg else v
    i = int(np.searchsorted(vals, float(a)))
    cands = [j for j in (i - 1, i, i + 1) if 0 <= j < len(vals)]
    best = min(cands, key=lambda j: (abs(Fraction(vals[j]) - a), bits[j] & 1))
    if a > Fraction(65504) + Fraction(16):  # beyond the halfway point to 65536: infinity
        return (0xFC00 if neg else 0x7C00)
    r = int(bits[best])
    return (r | 0x8000) if neg else r   # a negative value rounding to zero is -0


def test_f16_fma_and_mul_are_single_rounding(orc):
    rng = np.random.default_rng(2)
    for _ in range(3000):
        a, b, c = (int(x) for x in rng.integers(0, 0x7C00, 3))
        a |= int(rng.integers(0, 2)) << 15
        c |= int(rng.integers(0, 2)) << 15
        fa, fb, fc = (Fraction(float(np.uint16(z).view(np.float16))) for z in (a, b, c))
        exact = fa * fb + fc
        got = orc.lib().orc_f16_fma(a, b, c)
        if exact == 0:
            assert got in (0, 0x8000)
        else:
            assert got == _round_f16_exact(exact), (hex(a), hex(b), hex(c), hex(got))
        want_m = _round_f16_exact(fa * fb) if fa * fb != 0 else None
        got_m = orc.lib().orc_f16_mul(a, b)
        if want_m is not None:
            assert got_m == want_m


# ------------------------------------------------------------------------------------------------ Q4_K layout
def _pack_scales(sc, m):
    """the GGUF K-quant scale bytes from 8 six-bit scales and mins: bytes 0-3 low 6 bits sc0-3, bytes 4-7 low 6 bits
    m0-3, bytes 8-11 low nibble sc4-7 / high nibble m4-7, the high 2 bits of sc4-7 / m4-7 in the top bits of bytes
    0-3 / 4-7"""
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return bytes(s)


def test_q4k_scale_min_decodes_every_slot(orc):
    import ctypes
    rng = np.random.default_rng(3)
    for _ in range(300):
        sc = rng.integers(0, 64, 8).tolist()
        m = rng.integers(0, 64, 8).tolist()
        buf = (ctypes.c_uint8 * 12).from_buffer_copy(_pack_scales(sc, m))
        for j in range(8):
            a, b = ctypes.c_int(), ctypes.c_int()
            orc.lib().orc_q4k_scale_min(ctypes.addressof(buf), j, ctypes.addressof(a), ctypes.addressof(b))
            assert (a.value, b.value) == (sc[j], m[j])


def _q4k_block(d_bits, dmin_bits, sc, m, q):
    """a Q4_K block: q[j][l] is value l of sub-block j; sub-blocks 2i / 2i+1 share bytes 32 i .. 32 i + 31 as low /
    high nibbles"""
    qs = bytearray(128)
    for j in range(8):
        for l in range(32):
            qs[32 * (j // 2) + l] |= (q[j][l] & 15) << (4 * (j % 2))
    return np.frombuffer(np.uint16([d_bits, dmin_bits]).tobytes() + _pack_scales(sc, m) + bytes(qs), np.uint8)


def test_q4k_dequant_known_block(orc):
    sc = [1, 2, 3, 63, 17, 40, 0, 5]
    m = [0, 1, 7, 63, 32, 9, 2, 44]
    q = [[(l + 3 * j) % 16 for l in range(32)] for j in range(8)]
    blk = _q4k_block(0x3C00, 0x3800, sc, m, q)  # d = 1, dmin = 0.5
    got = orc.dequant(orc.Q4_K, blk, 1, 256)[0]
    want = np.array([sc[j] * q[j][l] - 0.5 * m[j] for j in range(8) for l in range(32)], np.float32)
    assert np.array_equal(got, want)
    # the tensor-core form: f16(q * f16(d sc) - f16(dmin m)); exact here
    got16 = orc.dequant_f16(orc.Q4_K, blk, 1, 256)[0].view(np.float16).astype(np.float32)
    assert np.array_equal(got16, want)


def test_q4k_dequant_f16_rounds_once(orc):
    rng = np.random.default_rng(4)
    sc = rng.integers(0, 64, 8).tolist()
    m = rng.integers(0, 64, 8).tolist()
    q = rng.integers(0, 16, (8, 32)).tolist()
    blk = _q4k_block(0x1E66, 0x1A3D, sc, m, q)
    d, dmin = (Fraction(float(np.uint16(b).view(np.float16))) for b in (0x1E66, 0x1A3D))
    got = orc.dequant_f16(orc.Q4_K, blk, 1, 256)[0]
    for j in range(8):
        d1 = Fraction(float(np.float16(np.float32(float(d * sc[j])))))
        nm1 = Fraction(float(np.float16(np.float32(-float(dmin * m[j])))))
        for l in range(32):
            assert got[32 * j + l] == _round_f16_exact(q[j][l] * d1 + nm1) or q[j][l] * d1 + nm1 == 0


def test_q8_0_dequant_known_block(orc):
    q = np.arange(-16, 16, dtype=np.int8)
    blk = np.frombuffer(np.uint16([0x3400]).tobytes() + q.tobytes(), np.uint8)  # d = 0.25
    assert np.array_equal(orc.dequant(orc.Q8_0, blk, 1, 32)[0], q.astype(np.float32) * 0.25)
    assert np.array_equal(orc.dequant_f16(orc.Q8_0, blk, 1, 32)[0].view(np.float16).astype(np.float32),
                          q.astype(np.float32) * 0.25)


# ------------------------------------------------------------------------------------------------ quantizers
def test_q4k_quantizer_round_trip_bound(orc):
    rows, cols = 64, 1024
    x = orc.synth(rows * cols, 11, 0.02).reshape(rows, cols)
    blk = orc.quantize(orc.Q4_K, x)
    y = orc.dequant(orc.Q4_K, blk, rows, cols)
    xs = x.reshape(-1, 8, 32).astype(np.float64)
    ys = y.reshape(-1, 8, 32).astype(np.float64)
    hdr = blk.reshape(-1, 144)[:, :4].copy().view(np.float16).astype(np.float64)  # d, dmin per super-block
    mn = np.minimum(xs.min(axis=2), 0.0)
    scale = (xs.max(axis=2) - mn) / 15
    import ctypes
    for k in range(xs.shape[0]):
        s12 = (ctypes.c_uint8 * 12).from_buffer_copy(blk.reshape(-1, 144)[k, 4:16].tobytes())
        for j in range(8):
            a, b = ctypes.c_int(), ctypes.c_int()
            orc.lib().orc_q4k_scale_min(ctypes.addressof(s12), j, ctypes.addressof(a), ctypes.addressof(b))
            assert 0 <= a.value < 64 and 0 <= b.value < 64
            dl, ml = hdr[k, 0] * a.value, hdr[k, 1] * b.value
            bound = 0.5 * dl + 15 * abs(scale[k, j] - dl) + 2 * abs(ml + mn[k, j]) + 1e-7
            assert np.max(np.abs(xs[k, j] - ys[k, j])) <= bound
    rel = np.sqrt(np.mean((x - y) ** 2)) / np.std(x)
    assert rel < 0.12, rel


def test_q4k_quantizer_is_exact_on_its_own_grid(orc):
    """values already on a block's grid (d sc q - dmin m with q spanning 0..15 in every sub-block) come back bit-exact"""
    rng = np.random.default_rng(5)
    for _ in range(20):
        sc = rng.integers(1, 64, 8)
        sc[int(rng.integers(0, 8))] = 63
        q = rng.integers(0, 16, (8, 32))
        q[:, 0], q[:, 1] = 0, 15
        blk = _q4k_block(0x1400, 0x0000, sc.tolist(), [0] * 8, q.tolist())
        x = orc.dequant(orc.Q4_K, blk, 1, 256)
        back = orc.quantize(orc.Q4_K, x)
        assert np.array_equal(orc.dequant(orc.Q4_K, back, 1, 256), x)


def test_q8_0_quantizer_known_answers(orc):
    x = np.zeros(32, np.float32)
    x[:6] = [127, -63.5, 0.5, 0.49, -0.5, 2.5]   # amax 127: d = 1, round half away from zero
    blk = orc.quantize(orc.Q8_0, x.reshape(1, 32))
    q = blk[2:].view(np.int8)
    assert blk[:2].view(np.uint16)[0] == 0x3C00
    assert q[:6].tolist() == [127, -64, 1, 0, -1, 3] and not q[6:].any()
    z = orc.quantize(orc.Q8_0, np.zeros((1, 32), np.float32))
    assert not z.any()


def test_q8_0_quantizer_bound(orc):
    x = orc.synth(4096, 12, 1.0).reshape(128, 32)
    blk = orc.quantize(orc.Q8_0, x).reshape(128, 34)
    d32 = np.abs(x).max(axis=1) / np.float32(127)
    q = blk[:, 2:].view(np.int8).astype(np.float64)
    assert np.all(np.abs(x / d32[:, None] - q) <= 0.5 + 1e-5)
    assert np.all(np.abs(q).max(axis=1) == 127)


# ------------------------------------------------------------------------------------------------ q8_1
def test_q8_1_known_block(orc):
    x = np.zeros((2, 32), np.float32)
    x[0, :5] = [63.5, 0.25, -0.25, 0.75, -63.5]   # amax 63.5: d = 0.5, x / d = 127, 0.5, -0.5, 1.5, -127
    q = orc.quantize_q8_1(x).reshape(2, 36)
    assert q[0, :2].view(np.uint16)[0] == 0x3800 and q[0, 2:4].view(np.uint16)[0] == np.float16(0.75).view(np.uint16)
    assert q[0, 4:9].view(np.int8).tolist() == [127, 1, -1, 2, -127] and not q[0, 9:].any()
    assert not q[1].any()   # an all-zero block: d 0, sum 0, q 0


def test_q8_1_bounds_and_sum(orc):
    x = orc.synth(8 * 2048, 13, 1.0).reshape(8, 2048)
    q = orc.quantize_q8_1(x).reshape(8, 64, 36)
    d = q[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    s = q[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    qs = q[..., 4:].view(np.int8).astype(np.float64)
    xb = x.reshape(8, 64, 32).astype(np.float64)
    d32 = np.abs(xb).max(axis=2) / 127
    assert np.all(np.abs(xb / d32[..., None] - qs) <= 0.5 + 1e-5)
    assert np.allclose(d, d32, rtol=1e-3)
    assert np.allclose(s, xb.sum(axis=2), rtol=2e-3, atol=2e-3)


# ------------------------------------------------------------------------------------------------ Q5_K
def _q5k_block(d_bits, dmin_bits, sc, m, q):
    """a Q5_K block (ggml block_q5_K): q[j][l] (0..31) is value l of sub-block j; its low 4 bits go where Q4_K keeps
    them (qs, after a 32-byte qh), its fifth bit is bit j of qh[l]"""
    qs = bytearray(128)
    qh = bytearray(32)
    for j in range(8):
        for l in range(32):
            qs[32 * (j // 2) + l] |= (q[j][l] & 15) << (4 * (j % 2))
            qh[l] |= (q[j][l] >> 4) << j
    return np.frombuffer(np.uint16([d_bits, dmin_bits]).tobytes() + _pack_scales(sc, m) + bytes(qh) + bytes(qs), np.uint8)


def test_q5k_dequant_known_block(orc):
    sc = [1, 2, 3, 63, 17, 40, 0, 5]
    m = [0, 1, 7, 63, 32, 9, 2, 44]
    # every sub-block uses all 32 values, each sub-block a different rotation so that a wrong qh bit index shows
    q = [[(l * 7 + 5 * j) % 32 for l in range(32)] for j in range(8)]
    blk = _q5k_block(0x3C00, 0x3800, sc, m, q)  # d = 1, dmin = 0.5
    assert blk.size == 176
    got = orc.dequant(orc.Q5_K, blk, 1, 256)[0]
    want = np.array([sc[j] * q[j][l] - 0.5 * m[j] for j in range(8) for l in range(32)], np.float32)
    assert np.array_equal(got, want)
    # the tensor-core form rounds the exact q f16(d sc) - f16(dmin m) once to f16 (above 1024 not every half is one)
    got16 = orc.dequant_f16(orc.Q5_K, blk, 1, 256)[0].view(np.float16)
    assert np.array_equal(got16, want.astype(np.float16))


def test_q5k_dequant_f16_rounds_once(orc):
    rng = np.random.default_rng(14)
    sc = rng.integers(0, 64, 8).tolist()
    m = rng.integers(0, 64, 8).tolist()
    q = rng.integers(0, 32, (8, 32)).tolist()
    blk = _q5k_block(0x1E66, 0x1A3D, sc, m, q)
    d, dmin = (Fraction(float(np.uint16(b).view(np.float16))) for b in (0x1E66, 0x1A3D))
    got = orc.dequant_f16(orc.Q5_K, blk, 1, 256)[0]
    for j in range(8):
        d1 = Fraction(float(np.float16(np.float32(float(d * sc[j])))))
        nm1 = Fraction(float(np.float16(np.float32(-float(dmin * m[j])))))
        for l in range(32):
            assert got[32 * j + l] == _round_f16_exact(q[j][l] * d1 + nm1) or q[j][l] * d1 + nm1 == 0


def test_q5k_quantizer_is_exact_on_its_own_grid(orc):
    """values on a block's grid (d sc q - dmin m with q spanning 0..31 in every sub-block) come back bit-exact"""
    rng = np.random.default_rng(15)
    for _ in range(20):
        sc = rng.integers(1, 64, 8)
        sc[int(rng.integers(0, 8))] = 63
        q = rng.integers(0, 32, (8, 32))
        q[:, 0], q[:, 1] = 0, 31
        blk = _q5k_block(0x1400, 0x0000, sc.tolist(), [0] * 8, q.tolist())
        x = orc.dequant(orc.Q5_K, blk, 1, 256)
        back = orc.quantize(orc.Q5_K, x)
        assert np.array_equal(back, blk)


def test_q5k_quantizer_round_trip_bound(orc):
    """per sub-block the error is at most half a step plus what the 6-bit scale and min cost; the 31-level grid
    halves Q4_K's error on the same data"""
    rows, cols = 32, 1024
    x = orc.synth(rows * cols, 11, 0.02).reshape(rows, cols)
    y5 = orc.dequant(orc.Q5_K, orc.quantize(orc.Q5_K, x), rows, cols)
    y4 = orc.dequant(orc.Q4_K, orc.quantize(orc.Q4_K, x), rows, cols)
    e5 = np.sqrt(np.mean((x - y5) ** 2)) / np.std(x)
    e4 = np.sqrt(np.mean((x - y4) ** 2)) / np.std(x)
    assert e5 < 0.06 and e5 < 0.6 * e4, (e5, e4)
    blk = orc.quantize(orc.Q5_K, x).reshape(-1, 176)
    hdr = blk[:, :4].copy().view(np.float16).astype(np.float64)
    xs, ys = x.reshape(-1, 8, 32).astype(np.float64), y5.reshape(-1, 8, 32).astype(np.float64)
    mn = np.minimum(xs.min(axis=2), 0.0)
    scale = (xs.max(axis=2) - mn) / 31
    import ctypes
    for k in range(xs.shape[0]):
        s12 = (ctypes.c_uint8 * 12).from_buffer_copy(blk[k, 4:16].tobytes())
        for j in range(8):
            a, b = ctypes.c_int(), ctypes.c_int()
            orc.lib().orc_q4k_scale_min(ctypes.addressof(s12), j, ctypes.addressof(a), ctypes.addressof(b))
            dl, ml = hdr[k, 0] * a.value, hdr[k, 1] * b.value
            bound = 0.5 * dl + 31 * abs(scale[k, j] - dl) + 2 * abs(ml + mn[k, j]) + 1e-7
            assert np.max(np.abs(xs[k, j] - ys[k, j])) <= bound


# ------------------------------------------------------------------------------------------------ Q4_0, Q5_1
def test_q4_0_dequant_known_block(orc):
    """value l in the low nibble of byte l, value l + 16 in its high nibble; (q - 8) d"""
    q = [(5 * l + 3) % 16 for l in range(32)]
    qs = bytes(q[l] | (q[l + 16] << 4) for l in range(16))
    blk = np.frombuffer(np.uint16([0x3400]).tobytes() + qs, np.uint8)   # d = 0.25
    want = (np.array(q, np.float32) - 8) * 0.25
    assert np.array_equal(orc.dequant(orc.Q4_0, blk, 1, 32)[0], want)
    assert np.array_equal(orc.dequant_f16(orc.Q4_0, blk, 1, 32)[0].view(np.float16).astype(np.float32), want)


def test_q4_0_quantizer_known_answers(orc):
    """tools/mtp_experts.py:29-41: d = (first value of largest magnitude) / -8, q = min(15, trunc(x / d + 8.5))"""
    d = 0.125
    q = np.array([(7 * l + 1) % 16 for l in range(32)])
    q[5] = 0                                     # the largest magnitude, -8 d: d comes back exactly
    x = ((q - 8) * d).astype(np.float32).reshape(1, 32)
    blk = orc.quantize(orc.Q4_0, x)
    assert blk[:2].copy().view(np.float16)[0] == np.float16(d)
    assert np.array_equal(orc.dequant(orc.Q4_0, blk, 1, 32), x)
    # +8 before -8 at equal magnitude: d = 8 / -8 = -1, +8 -> q 0 -> 8; -8 -> q 16, clamped to 15 -> -7
    x2 = np.zeros((1, 32), np.float32)
    x2[0, 3], x2[0, 9] = 8.0, -8.0
    y2 = orc.dequant(orc.Q4_0, orc.quantize(orc.Q4_0, x2), 1, 32)[0]
    assert y2[3] == 8.0 and y2[9] == -7.0 and y2[0] == 0.0


def test_q5_1_dequant_known_block(orc):
    """value l: low nibble of byte l (l < 16) or high nibble of byte l - 16, fifth bit qh bit l; d q + m"""
    q = [(11 * l + 4) % 32 for l in range(32)]
    qh = sum(((q[l] >> 4) & 1) << l for l in range(32))
    qs = bytes((q[l] & 15) | ((q[l + 16] & 15) << 4) for l in range(16))
    blk = np.frombuffer(np.uint16([0x3800, 0xC000]).tobytes() + np.uint32([qh]).tobytes() + qs, np.uint8)  # d 0.5, m -2
    want = np.array(q, np.float32) * 0.5 - 2.0
    assert blk.size == 24
    assert np.array_equal(orc.dequant(orc.Q5_1, blk, 1, 32)[0], want)
    assert np.array_equal(orc.dequant_f16(orc.Q5_1, blk, 1, 32)[0].view(np.float16).astype(np.float32), want)


def test_q5_1_quantizer_exact_on_its_grid_and_bounded(orc):
    """values m + q d (d a power of two, q spanning 0..31) come back exactly; on normal data the error is at most
    half a step plus the f16 rounding of d and m"""
    q = np.array([(13 * l + 2) % 32 for l in range(32)])
    q[0], q[1] = 0, 31
    x = (-1.5 + q * 0.0625).astype(np.float32).reshape(1, 32)
    blk = orc.quantize(orc.Q5_1, x)
    assert np.array_equal(orc.dequant(orc.Q5_1, blk, 1, 32), x)
    rows, cols = 16, 1024
    xr = orc.synth(rows * cols, 21, 0.02).reshape(rows, cols)
    b = orc.quantize(orc.Q5_1, xr).reshape(-1, 24)
    y = orc.dequant(orc.Q5_1, b.reshape(-1), rows, cols).reshape(-1, 32).astype(np.float64)
    xs = xr.reshape(-1, 32).astype(np.float64)
    d = (xs.max(axis=1) - xs.min(axis=1)) / 31
    dm = b[:, :4].copy().view(np.float16).astype(np.float64)
    bound = 0.5 * d + 31 * np.abs(dm[:, 0] - d) + np.abs(dm[:, 1] - xs.min(axis=1)) + 1e-9
    assert np.all(np.abs(xs - y).max(axis=1) <= bound)


def test_q4_0_quantizer_zero_block_sign(orc):
    """an all-zero block: d = x[0] / -8, so +0 data stores d = -0 and -0 data d = +0 (numpy's float32 arithmetic)"""
    for z, want in ((0.0, 0x8000), (-0.0, 0x0000)):
        x = np.full((1, 32), z, np.float32)
        blk = orc.quantize(orc.Q4_0, x)
        assert int(blk[:2].copy().view(np.uint16)[0]) == want
        assert np.all(blk[2:] == 0x88)
