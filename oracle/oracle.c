/*
 * CPU oracle for the quantized MoE layer.  TEST INFRASTRUCTURE ONLY (see oracle.h): never linked into the product.
 * Built with -ffp-contract=off so every float expression rounds exactly as written; fused steps call fmaf.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------------ f16 */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t) (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = s;
        else {   /* subnormal: m * 2^-24, exact in fp32 */
            float v = (float) m * 5.9604644775390625e-8f;
            memcpy(&bits, &v, 4);
            bits |= s;
        }
    } else if (e == 31) bits = s | 0x7f800000u | (m << 13);
    else bits = s | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* round-to-nearest-even of sign * mag * 2^e to f16 */
static uint16_t f16_round(int neg, unsigned __int128 mag, int e) {
    const uint16_t sg = neg ? 0x8000u : 0u;
    if (mag == 0) return sg;
    const uint64_t hi = (uint64_t) (mag >> 64), lo = (uint64_t) mag;
    const int hb = hi ? 127 - __builtin_clzll(hi) : 63 - __builtin_clzll(lo);   /* the highest set bit */
    int q = hb + e - 10;   /* exponent of the result's last mantissa bit */
    if (q < -24) q = -24;
    const int shift = q - e;
    unsigned __int128 r;
    if (shift <= 0) r = mag << (-shift);
    else {
        r = mag >> shift;
        const unsigned __int128 rem = mag - (r << shift), half = (unsigned __int128) 1 << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) ++r;
    }
    if (r >= 2048) {   /* the rounding carried into a new bit */
        r >>= 1;
        ++q;
    }
    if (r < 1024) return (uint16_t) (sg | (uint16_t) r);   /* subnormal (q == -24) */
    const int E = q + 25;
    if (E >= 31) return (uint16_t) (sg | 0x7c00u);
    return (uint16_t) (sg | (uint16_t) (E << 10) | (uint16_t) (r & 0x3ffu));
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const int neg = (x >> 31) & 1;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t) ((neg ? 0x8000u : 0u) | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax == 0) return neg ? 0x8000u : 0u;
    const int ef = (int) (ax >> 23);
    const uint32_t m = ef ? ((ax & 0x7fffffu) | 0x800000u) : (ax & 0x7fffffu);
    return f16_round(neg, m, (ef ? ef : 1) - 150);
}

/* an f16 as sign, integer mantissa and exponent: |v| = M 2^E; returns 0 for inf / NaN */
static int f16_parts(uint16_t h, int* neg, int64_t* M, int* E) {
    const int e = (h >> 10) & 31, m = h & 0x3ff;
    *neg = (h >> 15) & 1;
    if (e == 31) return 0;
    if (e == 0) {
        *M = m;
        *E = -24;
    } else {
        *M = m | 0x400;
        *E = e - 25;
    }
    return 1;
}

uint16_t orc_f16_fma(uint16_t a, uint16_t b, uint16_t c) {
    int na, nb, nc, ea, eb, ec;
    int64_t ma, mb, mc;
    if (!f16_parts(a, &na, &ma, &ea) || !f16_parts(b, &nb, &mb, &eb) || !f16_parts(c, &nc, &mc, &ec))
        return orc_f32_to_f16(fmaf(orc_f16_to_f32(a), orc_f16_to_f32(b), orc_f16_to_f32(c)));
    const int np = na ^ nb, ep = ea + eb;
    const int64_t mp = ma * mb;
    if (mp == 0 && mc == 0) return (np && nc) ? 0x8000u : 0u;
    const int e0 = ep < ec ? ep : ec;
    __int128 sp = (__int128) mp << (ep - e0), sc = (__int128) mc << (ec - e0);
    if (np) sp = -sp;
    if (nc) sc = -sc;
    const __int128 s = sp + sc;
    if (s == 0) return 0u;   /* exact cancellation: +0 under round-to-nearest */
    return f16_round(s < 0, (unsigned __int128) (s < 0 ? -s : s), e0);
}

uint16_t orc_f16_mul(uint16_t a, uint16_t b) {
    int na, nb, ea, eb;
    int64_t ma, mb;
    if (!f16_parts(a, &na, &ma, &ea) || !f16_parts(b, &nb, &mb, &eb))
        return orc_f32_to_f16(orc_f16_to_f32(a) * orc_f16_to_f32(b));
    return f16_round(na ^ nb, (unsigned __int128) (ma * mb), ea + eb);
}

/* ------------------------------------------------------------------------------------------------ synthetic data */
static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static inline float synth_one(uint64_t seed, uint64_t i, float std) {
    int64_t s = 0;
    for (int m = 0; m < 6; ++m) {
        const uint64_t r = mix64(seed + (6 * i + (uint64_t) m + 1) * 0x9e3779b97f4a7c15ull);
        s += (int64_t) (r & 0xffffffu) + (int64_t) ((r >> 32) & 0xffffffu);
    }
    const float z = (float) (int32_t) (s - 6 * (1ll << 24)) * 5.9604644775390625e-8f;
    return z * std;
}
void orc_synth_normal(float* out, size_t n, uint64_t seed, uint64_t offset, float std) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t) n; ++i) out[i] = synth_one(seed, offset + (uint64_t) i, std);
}

/* ------------------------------------------------------------------------------------------------ weight formats */
void orc_q4k_scale_min(const uint8_t* s, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

/* the K-quant super-block of 256 values: Q4_K (q5 = 0: header, qs[128]) or Q5_K (q5 = 1: header, qh[32], qs[128]);
 * levels 15 or 31 */
static void quant_kq_block(const float* x, uint8_t* b, int q5) {
    const float levels = q5 ? 31.0f : 15.0f;
    const int qmax = q5 ? 31 : 15;
    float scale[8], mn8[8], max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; ++j) {
        float mn = x[32 * j], mx = x[32 * j];
        for (int l = 1; l < 32; ++l) {
            if (x[32 * j + l] < mn) mn = x[32 * j + l];
            if (x[32 * j + l] > mx) mx = x[32 * j + l];
        }
        if (mn > 0.f) mn = 0.f;
        scale[j] = (mx - mn) / levels;
        mn8[j] = mn < 0.f ? -mn : 0.f;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (mn8[j] > max_min) max_min = mn8[j];
    }
    const uint16_t dh = orc_f32_to_f16(max_scale / 63.0f), mh = orc_f32_to_f16(max_min / 63.0f);
    const float df = orc_f16_to_f32(dh), mf = orc_f16_to_f32(mh);
    int sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = df > 0.f ? clampi((int) roundf(scale[j] / df), 0, 63) : 0;
        m[j] = mf > 0.f ? clampi((int) roundf(mn8[j] / mf), 0, 63) : 0;
    }
    memcpy(b, &dh, 2);
    memcpy(b + 2, &mh, 2);
    uint8_t* s = b + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t) ((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t) ((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t) ((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t* qh = b + 16;
    uint8_t* qs = b + (q5 ? 48 : 16);
    memset(qs, 0, 128);
    if (q5) memset(qh, 0, 32);
    for (int j = 0; j < 8; ++j) {
        const float dl = df * (float) sc[j], ml = mf * (float) m[j];
        for (int l = 0; l < 32; ++l) {
            const int q = dl > 0.f ? clampi((int) roundf((x[32 * j + l] + ml) / dl), 0, qmax) : 0;
            qs[32 * (j / 2) + l] |= (uint8_t) ((q & 15) << (4 * (j % 2)));
            if (q5) qh[l] |= (uint8_t) ((q >> 4) << j);
        }
    }
}

void orc_quantize_q4_k(const float* x, void* dst, int64_t rows, int cols) {
    const int nb = cols / 256;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int b = 0; b < nb; ++b)
            quant_kq_block(x + r * cols + 256 * b, (uint8_t*) dst + (r * nb + b) * ORC_Q4K_BYTES, 0);
}

void orc_quantize_q5_k(const float* x, void* dst, int64_t rows, int cols) {
    const int nb = cols / 256;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int b = 0; b < nb; ++b)
            quant_kq_block(x + r * cols + 256 * b, (uint8_t*) dst + (r * nb + b) * ORC_Q5K_BYTES, 1);
}

void orc_quantize_q8_0(const float* x, void* dst, int64_t rows, int cols) {
    const int64_t nblk = rows * (cols / 32);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < nblk; ++k) {
        const float* v = x + 32 * k;
        uint8_t* b = (uint8_t*) dst + k * ORC_Q80_BYTES;
        float amax = 0.f;
        for (int l = 0; l < 32; ++l) amax = fabsf(v[l]) > amax ? fabsf(v[l]) : amax;
        const float d = amax / 127.0f, idv = d != 0.f ? 1.0f / d : 0.f;
        const uint16_t dh = orc_f32_to_f16(d);
        memcpy(b, &dh, 2);
        for (int l = 0; l < 32; ++l) {
            const float t = v[l] * idv;
            const float a = floorf(fabsf(t) + 0.5f);
            b[2 + l] = (uint8_t) (int8_t) (int) (t < 0.f ? -a : a);
        }
    }
}

/* tools/mtp_experts.py:29-41: d = (the first value of largest magnitude) / -8, q = min(15, trunc(x / d + 8.5)) with
 * 1 / d in fp32 from the unrounded d; f16 d, then value l in the low nibble of byte l, value l + 16 in its high nibble */
void orc_quantize_q4_0(const float* x, void* dst, int64_t rows, int cols) {
    const int64_t nblk = rows * (cols / 32);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < nblk; ++k) {
        const float* v = x + 32 * k;
        uint8_t* b = (uint8_t*) dst + k * ORC_Q40_BYTES;
        float amax = fabsf(v[0]), mx = v[0];   /* the first value of largest magnitude (numpy's argmax) */
        for (int l = 1; l < 32; ++l)
            if (fabsf(v[l]) > amax) {
                amax = fabsf(v[l]);
                mx = v[l];
            }
        const float d = mx / -8.0f, idv = d != 0.f ? 1.0f / d : 0.f;
        const uint16_t dh = orc_f32_to_f16(d);
        memcpy(b, &dh, 2);
        for (int l = 0; l < 16; ++l) {
            const float a = truncf(v[l] * idv + 8.5f), c = truncf(v[l + 16] * idv + 8.5f);
            const int q0 = (int) (a < 15.f ? a : 15.f), q1 = (int) (c < 15.f ? c : 15.f);
            b[2 + l] = (uint8_t) (q0 | (q1 << 4));
        }
    }
}

/* Q5_1 (ggml block_q5_1, 24 bytes: f16 d, f16 m, u32 qh, 16 bytes qs): the library's quantizer, ggml's closed form:
 * m = min, d = (max - min) / 31, q = trunc((x - m) / d + 0.5) with 1 / d in fp32; value l's fifth bit is qh bit l */
void orc_quantize_q5_1(const float* x, void* dst, int64_t rows, int cols) {
    const int64_t nblk = rows * (cols / 32);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < nblk; ++k) {
        const float* v = x + 32 * k;
        uint8_t* b = (uint8_t*) dst + k * ORC_Q51_BYTES;
        float mn = v[0], mx = v[0];
        for (int l = 1; l < 32; ++l) {
            if (v[l] < mn) mn = v[l];
            if (v[l] > mx) mx = v[l];
        }
        const float d = (mx - mn) / 31.0f, idv = d != 0.f ? 1.0f / d : 0.f;
        const uint16_t dh = orc_f32_to_f16(d), mh = orc_f32_to_f16(mn);
        memcpy(b, &dh, 2);
        memcpy(b + 2, &mh, 2);
        uint32_t qh = 0;
        for (int l = 0; l < 16; ++l) {
            const int q0 = (int) truncf((v[l] - mn) * idv + 0.5f), q1 = (int) truncf((v[l + 16] - mn) * idv + 0.5f);
            b[8 + l] = (uint8_t) ((q0 & 15) | ((q1 & 15) << 4));
            qh |= (uint32_t) ((q0 >> 4) & 1) << l;
            qh |= (uint32_t) ((q1 >> 4) & 1) << (l + 16);
        }
        memcpy(b + 4, &qh, 4);
    }
}

/* value l (0..31) of a Q4_0 (q - 8 comes later) or Q5_1 block */
static inline int b32_value(const uint8_t* p, int type, int l) {
    if (type == ORC_Q4_0) return l < 16 ? p[2 + l] & 15 : p[2 + l - 16] >> 4;
    uint32_t qh;
    memcpy(&qh, p + 4, 4);
    const int nib = l < 16 ? p[8 + l] & 15 : p[8 + l - 16] >> 4;
    return nib | (int) (((qh >> l) & 1) << 4);
}
static inline size_t b32_bytes(int type) { return type == ORC_Q4_0 ? ORC_Q40_BYTES : ORC_Q51_BYTES; }

/* fp32: Q4_0 (q - 8) d; Q5_1 d q + m (ggml's dequantize_row_q4_0 / _q5_1) */
static void dequant_b32(const void* src, float* y, int64_t rows, int cols, int type) {
    const int64_t nblk = rows * (cols / 32);
    for (int64_t k = 0; k < nblk; ++k) {
        const uint8_t* p = (const uint8_t*) src + k * b32_bytes(type);
        uint16_t dh, mh = 0;
        memcpy(&dh, p, 2);
        if (type == ORC_Q5_1) memcpy(&mh, p + 2, 2);
        const float d = orc_f16_to_f32(dh), m = orc_f16_to_f32(mh);
        for (int l = 0; l < 32; ++l)
            y[32 * k + l] = type == ORC_Q4_0 ? (float) (b32_value(p, type, l) - 8) * d : d * (float) b32_value(p, type, l) + m;
    }
}
/* f16: Q4_0 hmul2(q - 8, d); Q5_1 hfma2(q, d, m), src/moe_mma.cuh:137-173 */
static void dequant_b32_f16(const void* src, uint16_t* y, int64_t rows, int cols, int type) {
    const int64_t nblk = rows * (cols / 32);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < nblk; ++k) {
        const uint8_t* p = (const uint8_t*) src + k * b32_bytes(type);
        uint16_t dh, mh;
        memcpy(&dh, p, 2);
        memcpy(&mh, p + 2, 2);
        for (int l = 0; l < 32; ++l)
            y[32 * k + l] = type == ORC_Q4_0 ? orc_f16_mul(orc_f32_to_f16((float) (b32_value(p, type, l) - 8)), dh)
                                             : orc_f16_fma(orc_f32_to_f16((float) b32_value(p, type, l)), dh, mh);
    }
}
void orc_dequant_q4_0(const void* src, float* y, int64_t rows, int cols) { dequant_b32(src, y, rows, cols, ORC_Q4_0); }
void orc_dequant_q4_0_f16(const void* src, uint16_t* y, int64_t rows, int cols) { dequant_b32_f16(src, y, rows, cols, ORC_Q4_0); }
void orc_dequant_q5_1(const void* src, float* y, int64_t rows, int cols) { dequant_b32(src, y, rows, cols, ORC_Q5_1); }
void orc_dequant_q5_1_f16(const void* src, uint16_t* y, int64_t rows, int cols) { dequant_b32_f16(src, y, rows, cols, ORC_Q5_1); }

/* value l of sub-block j of a K-quant super-block (Q5_K: the fifth bit from qh[l] bit j) */
static inline int kq_value(const uint8_t* p, int q5, int j, int l) {
    const uint8_t* qs = p + (q5 ? 48 : 16);
    const int nib = (qs[32 * (j / 2) + l] >> (4 * (j % 2))) & 0xF;
    return q5 ? nib | (((p[16 + l] >> j) & 1) << 4) : nib;
}

static void dequant_kq(const void* src, float* y, int64_t rows, int cols, int q5) {
    const int64_t nblk = rows * (cols / 256);
    const size_t bb = q5 ? ORC_Q5K_BYTES : ORC_Q4K_BYTES;
    for (int64_t k = 0; k < nblk; ++k) {
        const uint8_t* p = (const uint8_t*) src + k * bb;
        uint16_t dh, mh;
        memcpy(&dh, p, 2);
        memcpy(&mh, p + 2, 2);
        const float d = orc_f16_to_f32(dh), dmin = orc_f16_to_f32(mh);
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            orc_q4k_scale_min(p + 4, j, &sc, &m);
            const float d1 = d * (float) sc, m1 = dmin * (float) m;
            for (int l = 0; l < 32; ++l) y[256 * k + 32 * j + l] = d1 * (float) kq_value(p, q5, j, l) - m1;
        }
    }
}

static void dequant_kq_f16(const void* src, uint16_t* y, int64_t rows, int cols, int q5) {
    const int64_t nblk = rows * (cols / 256);
    const size_t bb = q5 ? ORC_Q5K_BYTES : ORC_Q4K_BYTES;
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < nblk; ++k) {
        const uint8_t* p = (const uint8_t*) src + k * bb;
        uint16_t dh, mh;
        memcpy(&dh, p, 2);
        memcpy(&mh, p + 2, 2);
        const float d = orc_f16_to_f32(dh), dmin = orc_f16_to_f32(mh);
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            orc_q4k_scale_min(p + 4, j, &sc, &m);
            const uint16_t d1 = orc_f32_to_f16(d * (float) sc), nm1 = orc_f32_to_f16(-(dmin * (float) m));
            for (int l = 0; l < 32; ++l) {
                const uint16_t qh = orc_f32_to_f16((float) kq_value(p, q5, j, l));
                y[256 * k + 32 * j + l] = orc_f16_fma(qh, d1, nm1);
            }
        }
    }
}

void orc_dequant_q4_k(const void* src, float* y, int64_t rows, int cols) { dequant_kq(src, y, rows, cols, 0); }
void orc_dequant_q4_k_f16(const void* src, uint16_t* y, int64_t rows, int cols) { dequant_kq_f16(src, y, rows, cols, 0); }
void orc_dequant_q5_k(const void* src, float* y, int64_t rows, int cols) { dequant_kq(src, y, rows, cols, 1); }
void orc_dequant_q5_k_f16(const void* src, uint16_t* y, int64_t rows, int cols) { dequant_kq_f16(src, y, rows, cols, 1); }

void orc_dequant_q8_0(const void* src, float* y, int64_t rows, int cols) {
    const int64_t nblk = rows * (cols / 32);
    for (int64_t k = 0; k < nblk; ++k) {
        const uint8_t* p = (const uint8_t*) src + k * ORC_Q80_BYTES;
        uint16_t dh;
        memcpy(&dh, p, 2);
        const float d = orc_f16_to_f32(dh);
        for (int l = 0; l < 32; ++l) y[32 * k + l] = d * (float) (int8_t) p[2 + l];
    }
}

void orc_dequant_q8_0_f16(const void* src, uint16_t* y, int64_t rows, int cols) {
    const int64_t nblk = rows * (cols / 32);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < nblk; ++k) {
        const uint8_t* p = (const uint8_t*) src + k * ORC_Q80_BYTES;
        uint16_t dh;
        memcpy(&dh, p, 2);
        for (int l = 0; l < 32; ++l) y[32 * k + l] = orc_f16_mul(orc_f32_to_f16((float) (int8_t) p[2 + l]), dh);
    }
}

/* ------------------------------------------------------------------------------------------------ activations */
/* a xor butterfly over n lanes (n a power of two): every lane ends with the same value, lane 0's is returned */
static float butterfly_sum(const float* v, int n) {
    float a[64], b[64];
    memcpy(a, v, (size_t) n * sizeof(float));
    for (int o = n / 2; o; o >>= 1) {
        for (int l = 0; l < n; ++l) b[l] = a[l] + a[l ^ o];
        memcpy(a, b, (size_t) n * sizeof(float));
    }
    return a[0];
}

static void q8_1_block(const float* x, uint8_t* blk) {
    float amax = 0.f;
    for (int l = 0; l < 32; ++l) amax = fabsf(x[l]) > amax ? fabsf(x[l]) : amax;
    const float sum = butterfly_sum(x, 32);
    const float d = amax / 127.0f;
    for (int l = 0; l < 32; ++l) blk[4 + l] = (uint8_t) (int8_t) (amax == 0.f ? 0 : (int) roundf(x[l] / d));
    const uint16_t dh = orc_f32_to_f16(d), sh = orc_f32_to_f16(sum);
    memcpy(blk, &dh, 2);
    memcpy(blk + 2, &sh, 2);
}

void orc_quantize_q8_1(const float* x, void* q, int n, int rows) {
    for (int64_t r = 0; r < rows; ++r)
        for (int b = 0; b < n / 32; ++b) q8_1_block(x + r * n + 32 * b, (uint8_t*) q + (r * (n / 32) + b) * ORC_Q81_BYTES);
}

static inline float silu_(float x) { return x / (1.0f + expf(-x)); }
static inline float sigm_(float x) { return 1.0f / (1.0f + expf(-x)); }

void orc_swiglu_q8_1(const float* gu, int ff, void* hq) {
    float h[32];
    for (int b = 0; b < ff / 32; ++b) {
        for (int l = 0; l < 32; ++l) h[l] = silu_(gu[32 * b + l]) * gu[ff + 32 * b + l];
        q8_1_block(h, (uint8_t*) hq + (size_t) b * ORC_Q81_BYTES);
    }
}

/* ------------------------------------------------------------------------------------------------ routing */
static float router_dot(const float* w, const float* x, int H) {
    float lane[64];
    for (int l = 0; l < 64; ++l) {
        float a = 0.f;
        for (int c = l; c < H / 4; c += 64)
            for (int u = 0; u < 4; ++u) a = fmaf(w[4 * c + u], x[4 * c + u], a);
        lane[l] = a;
    }
    return butterfly_sum(lane, 64);
}

void orc_router_logits(const float* W, const float* x, float* logits, int T, int H, int L) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < L; ++r)
        for (int t = 0; t < T; ++t) logits[(size_t) t * L + r] = router_dot(W + (size_t) r * H, x + (size_t) t * H, H);
}

/* src/prefill.cu:1163 (the prompt path's router sgemm) in the matrix-core kernel's order (see oracle.h) */
static float router_dot_mm(const float* w, const float* x, int H) {
    const int KW = H / 8;
    float sum = 0.f;
    for (int s = 0; s < 8; ++s) {
        float p = 0.f;
        for (int j = 0; j < KW / 16; ++j)
            for (int i = 0; i < 4; ++i)
                for (int g = 0; g < 4; ++g) {
                    const int k = s * KW + 16 * j + 4 * g + i;
                    p = fmaf(x[k], w[k], p);
                }
        sum = s == 0 ? p : sum + p;
    }
    return sum;
}

void orc_router_logits_mm(const float* W, const float* x, float* logits, int T, int H, int L) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < L; ++r)
        for (int t = 0; t < T; ++t) logits[(size_t) t * L + r] = router_dot_mm(W + (size_t) r * H, x + (size_t) t * H, H);
}

void orc_router_logits_prompt(const float* W, const float* x, float* logits, int T, int H, int L) {
    if (T >= ORC_ROUTER_MM_MIN_T) orc_router_logits_mm(W, x, logits, T, H, L);
    else orc_router_logits(W, x, logits, T, H, L);
}

int orc_topk(const float* logits, int T, int E, int ld, int K, int* topi, float* topw) {
    int missing = 0;
    unsigned char* taken = (unsigned char*) malloc((size_t) E);
    for (int t = 0; t < T; ++t) {
        const float* v = logits + (size_t) t * ld;
        memset(taken, 0, (size_t) E);
        float top0 = 0.f, z = 0.f, ek[64];
        for (int k = 0; k < K; ++k) {
            float bv = -INFINITY;
            int bi = -1;
            for (int i = 0; i < E; ++i)
                if (!taken[i] && v[i] > bv) {
                    bv = v[i];
                    bi = i;
                }
            topi[t * K + k] = bi;
            if (bi < 0) {
                ek[k] = 0.f;
                ++missing;
                continue;
            }
            taken[bi] = 1;
            if (k == 0) top0 = bv;
            ek[k] = expf(bv - top0);
            z += ek[k];
        }
        for (int k = 0; k < K; ++k) topw[t * K + k] = topi[t * K + k] < 0 ? 0.f : ek[k] / z;
    }
    free(taken);
    return missing;
}

int orc_jobs_decode(const int* topi, int T, int K, int E, int shared, orc_job* gu, orc_job* dn) {
    int nj = 0;
    for (int p = 0; p < T * K; ++p) {
        const int e = topi[p];
        if (e < 0) continue;
        int j = 0;
        while (j < nj && gu[j].w != e) ++j;
        if (j == nj) {
            memset(&gu[j], 0, sizeof(orc_job));
            memset(&dn[j], 0, sizeof(orc_job));
            gu[j].w = dn[j].w = e;
            ++nj;
        }
        const int s = gu[j].n++;
        dn[j].n++;
        gu[j].y[s] = p / K;
        gu[j].out[s] = dn[j].y[s] = dn[j].out[s] = p;
    }
    if (shared) {
        memset(&gu[nj], 0, sizeof(orc_job));
        memset(&dn[nj], 0, sizeof(orc_job));
        gu[nj].w = dn[nj].w = E;
        gu[nj].n = dn[nj].n = T;
        for (int t = 0; t < T; ++t) {
            gu[nj].y[t] = t;
            gu[nj].out[t] = dn[nj].y[t] = dn[nj].out[t] = T * K + t;
        }
        ++nj;
    }
    return nj;
}

int orc_jobs_prefill(const int* topi, int C, int K, int E, int shared, int* cnt, int* jbase, orc_bigjob* gu,
                     orc_bigjob* dn) {
    const int P = C * K;
    memset(cnt, 0, (size_t) E * sizeof(int));
    for (int p = 0; p < P; ++p)
        if (topi[p] >= 0) cnt[topi[p]]++;
    int acc = 0;
    for (int e = 0; e < E; ++e) {
        jbase[e] = acc;
        acc += (cnt[e] + ORC_PF_JOB - 1) / ORC_PF_JOB;
    }
    int* fill = (int*) calloc((size_t) E, sizeof(int));
    for (int p = 0; p < P; ++p) {
        const int e = topi[p];
        if (e < 0) continue;
        const int s = fill[e]++, j = jbase[e] + s / ORC_PF_JOB, k = s % ORC_PF_JOB;
        if (k == 0) {
            memset(&gu[j], 0, sizeof(orc_bigjob));
            memset(&dn[j], 0, sizeof(orc_bigjob));
            gu[j].w = dn[j].w = e;
            gu[j].n = dn[j].n = cnt[e] - (s / ORC_PF_JOB) * ORC_PF_JOB < ORC_PF_JOB ? cnt[e] - (s / ORC_PF_JOB) * ORC_PF_JOB
                                                                                    : ORC_PF_JOB;
        }
        gu[j].y[k] = p / K;
        gu[j].out[k] = p;
        dn[j].y[k] = p;
        dn[j].out[k] = p;
    }
    free(fill);
    if (shared)
        for (int t0 = 0; t0 < C; t0 += ORC_PF_JOB) {
            const int j = acc++;
            memset(&gu[j], 0, sizeof(orc_bigjob));
            memset(&dn[j], 0, sizeof(orc_bigjob));
            gu[j].w = dn[j].w = E;
            gu[j].n = dn[j].n = C - t0 < ORC_PF_JOB ? C - t0 : ORC_PF_JOB;
            for (int k = 0; k < gu[j].n; ++k) {
                gu[j].y[k] = t0 + k;
                gu[j].out[k] = dn[j].y[k] = dn[j].out[k] = P + t0 + k;
            }
        }
    return acc;
}

/* ------------------------------------------------------------------------------------------------ expert dots */
/* group jg (sub-blocks 2 jg, 2 jg + 1) of a K-quant super-block against those two q8_1 blocks, src/moe_q4k.cuh:44-73
 * (Q5_K: the same combine on 5-bit values) */
static float kq_group_term(const uint8_t* blk, int q5, int jg, const uint8_t* ya, const uint8_t* yb) {
    uint16_t dh, mh, d8a, d8b;
    memcpy(&dh, blk, 2);
    memcpy(&mh, blk + 2, 2);
    memcpy(&d8a, ya, 2);
    memcpy(&d8b, yb, 2);
    const float d = orc_f16_to_f32(dh), dmin = orc_f16_to_f32(mh);
    int sc0i, m0i, sc1i, m1i;
    orc_q4k_scale_min(blk + 4, 2 * jg, &sc0i, &m0i);
    orc_q4k_scale_min(blk + 4, 2 * jg + 1, &sc1i, &m1i);
    const float sc0 = (float) sc0i, m0 = (float) m0i, sc1 = (float) sc1i, m1 = (float) m1i;
    int dl = 0, dhi = 0, sl = 0, sh = 0;
    for (int l = 0; l < 32; ++l) {
        const int al = (int8_t) ya[4 + l], ah = (int8_t) yb[4 + l];
        dl += kq_value(blk, q5, 2 * jg, l) * al;
        dhi += kq_value(blk, q5, 2 * jg + 1, l) * ah;
        sl += al;
        sh += ah;
    }
    const float d8l = orc_f16_to_f32(d8a), d8h = orc_f16_to_f32(d8b);
    return d * (d8l * (sc0 * (float) dl) + d8h * (sc1 * (float) dhi)) -
           dmin * (d8l * (m0 * (float) sl) + d8h * (m1 * (float) sh));
}

/* 8 lanes, lane l8 the groups l8 + 8 i in order, then the xor butterfly (src/moe_q4k.cuh:30-86, src/moe.cuh:224-235) */
static float dot_kq(const uint8_t* wrow, const uint8_t* yq, int K, int q5) {
    const int gpl = K / 64 / 8;
    const size_t bb = q5 ? ORC_Q5K_BYTES : ORC_Q4K_BYTES;
    float lane[8];
    for (int l8 = 0; l8 < 8; ++l8) {
        float tmp = 0.f;
        for (int i = 0; i < gpl; ++i) {
            const int g = l8 + 8 * i, b = g >> 2, jg = g & 3;
            const uint8_t* ya = yq + (size_t) (b * 8 + jg * 2) * ORC_Q81_BYTES;
            tmp += kq_group_term(wrow + (size_t) b * bb, q5, jg, ya, ya + ORC_Q81_BYTES);
        }
        lane[l8] = tmp;
    }
    return butterfly_sum(lane, 8);
}
float orc_dot_q4_k(const uint8_t* wrow, const uint8_t* yq, int K) { return dot_kq(wrow, yq, K, 0); }
float orc_dot_q5_k(const uint8_t* wrow, const uint8_t* yq, int K) { return dot_kq(wrow, yq, K, 1); }

float orc_dot_q8_0(const uint8_t* wrow, const uint8_t* yq, int K) {
    const int nb = K / 32;
    float lane[16];
    for (int l = 0; l < 16; ++l) {
        float acc = 0.f;
        for (int b = l; b < nb; b += 16) {
            const uint8_t* w = wrow + (size_t) b * ORC_Q80_BYTES;
            const uint8_t* a = yq + (size_t) b * ORC_Q81_BYTES;
            uint16_t dw, da;
            memcpy(&dw, w, 2);
            memcpy(&da, a, 2);
            int s = 0;
            for (int k = 0; k < 32; ++k) s += (int) (int8_t) w[2 + k] * (int) (int8_t) a[4 + k];
            acc += (orc_f16_to_f32(dw) * orc_f16_to_f32(da)) * (float) s;
        }
        lane[l] = acc;
    }
    return butterfly_sum(lane, 16);
}

/* Q4_0 / Q5_1 x q8_1: 16 lanes, lane l the blocks l + 16 i in order, then the xor butterfly (the Q8_0 lanes).  Per
 * block, with s = the integer sum of the activation block's int8 values: Q4_0 (d_w d_a) (sum q a - 8 s), i.e. the
 * exact integer sum (q - 8) a; Q5_1 (d_w d_a) sum q a + (m_w d_a) s.  (The reference's ggml vec_dot_q4_0_q8_1 /
 * _q5_1_q8_1 use the f16 block sum of the activations instead of d_a s: their bits are parity unpinned; these forms
 * are pinned by float64 products.) */
static float dot_b32(const uint8_t* wrow, const uint8_t* yq, int K, int type) {
    const int nb = K / 32;
    float lane[16];
    for (int l = 0; l < 16; ++l) {
        float acc = 0.f;
        for (int b = l; b < nb; b += 16) {
            const uint8_t* w = wrow + (size_t) b * b32_bytes(type);
            const uint8_t* a = yq + (size_t) b * ORC_Q81_BYTES;
            uint16_t dw, mw, da;
            memcpy(&dw, w, 2);
            memcpy(&mw, w + 2, 2);
            memcpy(&da, a, 2);
            int si = 0, sa = 0;
            for (int k = 0; k < 32; ++k) {
                si += b32_value(w, type, k) * (int) (int8_t) a[4 + k];
                sa += (int) (int8_t) a[4 + k];
            }
            const float dd = orc_f16_to_f32(dw) * orc_f16_to_f32(da);
            if (type == ORC_Q4_0) acc += dd * (float) (si - 8 * sa);
            else acc += dd * (float) si + (orc_f16_to_f32(mw) * orc_f16_to_f32(da)) * (float) sa;
        }
        lane[l] = acc;
    }
    return butterfly_sum(lane, 16);
}
float orc_dot_q4_0(const uint8_t* wrow, const uint8_t* yq, int K) { return dot_b32(wrow, yq, K, ORC_Q4_0); }
float orc_dot_q5_1(const uint8_t* wrow, const uint8_t* yq, int K) { return dot_b32(wrow, yq, K, ORC_Q5_1); }

/* The shared expert's dense Q8_0 rows, src/dense.cuh:24-154 q8s_block: 32 lanes, lane l the 16-column halves
 * c = 16 l + 512 i in order, acc = fmaf(d_w d_a, dot of the 16 values, acc), then the xor butterfly 16, 8, 4, 2, 1
 * (v += shfl_xor(v, o), src/dense.cuh:141-145).  d_a is the q8_1 block's f16 scale (its ds.x; the f16-rounded td
 * of the SwiGLU rows for the down projection). */
float orc_dot_q8s(const uint8_t* wrow, const uint8_t* yq, int K) {
    float lane[32];
    for (int l = 0; l < 32; ++l) {
        float acc = 0.f;
        for (int c = 16 * l; c < K; c += 512) {
            const int b = c / 32, half = (c / 16) & 1;
            const uint8_t* w = wrow + (size_t) b * ORC_Q80_BYTES;
            const uint8_t* a = yq + (size_t) b * ORC_Q81_BYTES;
            uint16_t dw, da;
            memcpy(&dw, w, 2);
            memcpy(&da, a, 2);
            int s = 0;
            for (int k = 0; k < 16; ++k) s += (int) (int8_t) w[2 + 16 * half + k] * (int) (int8_t) a[4 + 16 * half + k];
            acc = fmaf(orc_f16_to_f32(dw) * orc_f16_to_f32(da), (float) s, acc);
        }
        lane[l] = acc;
    }
    return butterfly_sum(lane, 32);
}

float orc_dot(int type, const uint8_t* wrow, const uint8_t* yq, int K) {
    switch (type) {
        case ORC_Q4_K: return orc_dot_q4_k(wrow, yq, K);
        case ORC_Q5_K: return orc_dot_q5_k(wrow, yq, K);
        case ORC_Q4_0: return orc_dot_q4_0(wrow, yq, K);
        case ORC_Q5_1: return orc_dot_q5_1(wrow, yq, K);
        default: return orc_dot_q8_0(wrow, yq, K);
    }
}

static size_t row_bytes(int type, int cols) {
    switch (type) {
        case ORC_Q4_K: return (size_t) cols / 256 * ORC_Q4K_BYTES;
        case ORC_Q5_K: return (size_t) cols / 256 * ORC_Q5K_BYTES;
        case ORC_Q4_0: return (size_t) cols / 32 * ORC_Q40_BYTES;
        case ORC_Q5_1: return (size_t) cols / 32 * ORC_Q51_BYTES;
        default: return (size_t) cols / 32 * ORC_Q80_BYTES;
    }
}

/* ------------------------------------------------------------------------------------------------ the layer */
static void layer_impl(const orc_layer* L, const float* x, int T, float* y, float* logits_out, int* topi_out,
                       float* topw_out, float* gu_out, float* part_out, int nthreads, int prompt) {
    const int H = L->H, E = L->E, K = L->K, ff = L->ff, P = T * K, NP = P + (L->shared ? T : 0);
    const size_t gurb = row_bytes(L->type, H), dnrb = row_bytes(L->dn_type, ff);
    uint8_t* xq = (uint8_t*) malloc((size_t) T * (H / 32) * ORC_Q81_BYTES);
    float* logits = logits_out ? logits_out : (float*) malloc((size_t) T * (E + 1) * sizeof(float));
    int* topi = topi_out ? topi_out : (int*) malloc((size_t) P * sizeof(int));
    float* topw = topw_out ? topw_out : (float*) malloc((size_t) P * sizeof(float));
    float* gu = gu_out ? gu_out : (float*) malloc((size_t) NP * 2 * ff * sizeof(float));
    float* part = part_out ? part_out : (float*) malloc((size_t) NP * H * sizeof(float));
    uint8_t* hq = (uint8_t*) malloc((size_t) NP * (ff / 32) * ORC_Q81_BYTES);
    int* pe = (int*) malloc((size_t) NP * sizeof(int));
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
    orc_quantize_q8_1(x, xq, H, T);
#pragma omp parallel for schedule(static) if (nthreads > 1)
    for (int r = 0; r < E + 1; ++r)
        for (int t = 0; t < T; ++t)
            logits[(size_t) t * (E + 1) + r] = prompt && T >= ORC_ROUTER_MM_MIN_T ? router_dot_mm(L->W + (size_t) r * H, x + (size_t) t * H, H)
                                                      : router_dot(L->W + (size_t) r * H, x + (size_t) t * H, H);
    orc_topk(logits, T, E, E + 1, K, topi, topw);
    for (int p = 0; p < NP; ++p) pe[p] = p < P ? topi[p] : E;
    const int64_t ngu = (int64_t) NP * 2 * ff;
#pragma omp parallel for schedule(static) if (nthreads > 1)
    for (int64_t q = 0; q < ngu; ++q) {
        const int p = (int) (q / (2 * ff)), r = (int) (q % (2 * ff)), t = p < P ? p / K : p - P;
        if (pe[p] < 0) continue;
        const uint8_t* xt = xq + (size_t) t * (H / 32) * ORC_Q81_BYTES;
        if (L->sh_gu && p >= P) gu[q] = orc_dot_q8s(L->sh_gu + (size_t) r * row_bytes(ORC_Q8_0, H), xt, H);
        else gu[q] = orc_dot(L->type, L->gu_w + (size_t) pe[p] * L->gu_stride + (size_t) r * gurb, xt, H);
    }
    for (int p = 0; p < NP; ++p)
        if (pe[p] >= 0) orc_swiglu_q8_1(gu + (size_t) p * 2 * ff, ff, hq + (size_t) p * (ff / 32) * ORC_Q81_BYTES);
    const int64_t ndn = (int64_t) NP * H;
#pragma omp parallel for schedule(static) if (nthreads > 1)
    for (int64_t q = 0; q < ndn; ++q) {
        const int p = (int) (q / H), r = (int) (q % H);
        if (pe[p] < 0) continue;
        const uint8_t* hp = hq + (size_t) p * (ff / 32) * ORC_Q81_BYTES;
        if (L->sh_dn && p >= P) part[q] = orc_dot_q8s(L->sh_dn + (size_t) r * row_bytes(ORC_Q8_0, ff), hp, ff);
        else part[q] = orc_dot(L->dn_type, L->dn_w + (size_t) pe[p] * L->dn_stride + (size_t) r * dnrb, hp, ff);
    }
    for (int t = 0; t < T; ++t) {
        const float g = L->shared ? sigm_(logits[(size_t) t * (E + 1) + E]) : 0.f;
        for (int i = 0; i < H; ++i) {
            float s = 0.f;
            for (int k = 0; k < K; ++k)
                if (topi[t * K + k] >= 0) s = fmaf(topw[t * K + k], part[(size_t) (t * K + k) * H + i], s);
            y[(size_t) t * H + i] = L->shared ? fmaf(g, part[(size_t) (P + t) * H + i], s) : s;
        }
    }
    free(xq);
    free(hq);
    free(pe);
    if (!logits_out) free(logits);
    if (!topi_out) free(topi);
    if (!topw_out) free(topw);
    if (!gu_out) free(gu);
    if (!part_out) free(part);
}

/* ------------------------------------------------------------------------------------------------ f16 path */
void orc_mma_matvec(const uint8_t* w, int type, int n_in, int n_out, const uint16_t* x16, double* out) {
    /* the whole matrix dequantized at once (the dequantizers split rows over threads), then one float64 sum a row */
    uint16_t* m = (uint16_t*) malloc((size_t) n_in * n_out * 2);
    if (type == ORC_Q4_K) orc_dequant_q4_k_f16(w, m, n_out, n_in);
    else if (type == ORC_Q5_K) orc_dequant_q5_k_f16(w, m, n_out, n_in);
    else if (type == ORC_Q4_0) orc_dequant_q4_0_f16(w, m, n_out, n_in);
    else if (type == ORC_Q5_1) orc_dequant_q5_1_f16(w, m, n_out, n_in);
    else orc_dequant_q8_0_f16(w, m, n_out, n_in);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n_out; ++r) {
        const uint16_t* row = m + (size_t) r * n_in;
        double s = 0.0;
        for (int k = 0; k < n_in; ++k) s += (double) orc_f16_to_f32(row[k]) * (double) orc_f16_to_f32(x16[k]);
        out[r] = s;
    }
    free(m);
}

void orc_swiglu_h16(const float* gu, int ff, uint16_t* h16) {
    for (int i = 0; i < ff; ++i) h16[i] = orc_f32_to_f16(silu_(gu[i]) * gu[ff + i]);
}

/* ------------------------------------------------------------------------------------------------ CPU baseline */
static double now_us(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double) ts.tv_sec * 1e6 + (double) ts.tv_nsec * 1e-3;
}
static int cmp_d(const void* a, const void* b) {
    const double x = *(const double*) a, y = *(const double*) b;
    return x < y ? -1 : x > y;
}

void orc_layer_decode(const orc_layer* L, const float* x, int T, float* y, float* logits, int* topi, float* topw,
                      float* gu, float* part, int nthreads) {
    layer_impl(L, x, T, y, logits, topi, topw, gu, part, nthreads, 0);
}
void orc_layer_prompt(const orc_layer* L, const float* x, int T, float* y, float* logits, int* topi, float* topw,
                      float* gu, float* part, int nthreads) {
    layer_impl(L, x, T, y, logits, topi, topw, gu, part, nthreads, 1);
}
double orc_time_layer_decode(const orc_layer* L, const float* x, int nthreads, int reps, size_t sweep_bytes, float* y) {
    double* t = (double*) malloc((size_t) reps * sizeof(double));
    uint64_t* sweep = sweep_bytes ? (uint64_t*) malloc(sweep_bytes) : NULL;
    if (sweep) memset(sweep, 1, sweep_bytes);
    volatile uint64_t sink = 0;
    for (int r = 0; r < reps; ++r) {
        if (sweep) {
            uint64_t s = 0;
#pragma omp parallel for reduction(+ : s) schedule(static)
            for (int64_t i = 0; i < (int64_t) (sweep_bytes / 8); i += 8) s += sweep[i];
            sink += s;
        }
        const double t0 = now_us();
        orc_layer_decode(L, x, 1, y, NULL, NULL, NULL, NULL, NULL, nthreads);
        t[r] = now_us() - t0;
    }
    (void) sink;
    qsort(t, (size_t) reps, sizeof(double), cmp_d);
    const double med = t[reps / 2];
    free(t);
    free(sweep);
    return med;
}

/* ------------------------------------------------------------------------------------------ hyper-connection read */
/* src/hc.cuh:13-380 k_hc (with hc_write's fold, src/kernels.cu:1493-1498, as its first step) for T rows, D = HC N
 * columns of HC residual streams, low rank LR.  Per row t:
 *   R' = R + bo * 2 sigm(inj_prev / HC) per stream (when bo), xs = R' w_norm;
 *   per 512-column slice s: the square sums of R' (32-lane butterflies, then the 16 groups in order: hc.cuh:165-180),
 *   xs as int8 per 32 (q8_block: float d = amax / 127, hc.cuh:60-66), and each down row's partial dot: 8 lanes, lane j
 *   the 8-value chunks q 8 + j in order, acc = fmaf(d_w d_x, dot8, acc), then xor 1, 2, 4 (hc.cuh:186-209); each
 *   bf16 inject row on xs itself (hc.cuh:211-226);
 *   rs_c = 1 / sqrt(sum of stream c's slice sums / N + eps); lo_r = silu(sum_c fmaf(rs_c, sum_s part) / HC) as int8
 *   per 32; inject_c likewise without silu (hc.cuh:251-289);
 *   up row c N + i: 16 lanes, lane b < LR / 32 the 32-block b, (d_w d_lo) dot32, xor 1, 2, 4, 8 (hc.cuh:318-344);
 *   mixed_i = sum_c sigm(up) ((R'_c,i w_norm) rs_c) / HC, then mixed as q8_1 (hc.cuh:346-381).
 * The reference's rsqrtf and __expf are approximations; here 1 / sqrtf and expf (parity of those bits unpinned). */
static inline float bf16_f(uint16_t h) {
    const uint32_t u = (uint32_t) h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static float butterfly_up(const float* v, int n) {   /* xor 1, 2, 4, ...: lane 0's value */
    float a[64], b[64];
    memcpy(a, v, (size_t) n * sizeof(float));
    for (int o = 1; o < n; o <<= 1) {
        for (int l = 0; l < n; ++l) b[l] = a[l] + a[l ^ o];
        memcpy(a, b, (size_t) n * sizeof(float));
    }
    return a[0];
}
static void q8_block_f(const float* x, int8_t* q, float* d) {   /* hc.cuh:60-66 */
    float amax = 0.f;
    for (int l = 0; l < 32; ++l) amax = fabsf(x[l]) > amax ? fabsf(x[l]) : amax;
    const float sc = amax / 127.0f;
    for (int l = 0; l < 32; ++l) q[l] = amax == 0.0f ? 0 : (int8_t) roundf(x[l] / sc);
    *d = sc;
}

void orc_hc_read(float* R, const float* bo, const float* inj_prev, const float* w_norm, const int8_t* dq,
                 const uint16_t* dd, const int8_t* uq, const uint16_t* ud, const uint16_t* w_inj, float eps, int T, int N,
                 int HC, int LR, float* mixed, float* inject, uint8_t* xq, float* part_out, float* ssp_out) {
    const int D = HC * N, NS = D / 512, SPS = N / 512, ROWS = LR + HC;
    float* Rp = (float*) malloc((size_t) D * sizeof(float));
    float* part = (float*) malloc((size_t) NS * ROWS * sizeof(float));
    float* ssp = (float*) malloc((size_t) NS * sizeof(float));
    float* lo = (float*) malloc((size_t) LR * sizeof(float));
    int8_t* loq = (int8_t*) malloc((size_t) LR);
    float lod[16], rs[64], gs[64];
    for (int t = 0; t < T; ++t) {
        for (int e = 0; e < D; ++e) {
            const int c = e / N, i = e % N;
            float r = R[(size_t) t * D + e];
            if (bo) r = fmaf(bo[(size_t) t * N + i], 2.0f * sigm_(inj_prev[t * HC + c] / (float) HC), r);
            Rp[e] = r;
        }
        for (int s = 0; s < NS; ++s) {
            const int col0 = s * 512;
            float xs[512], sq[32], xd[16];
            int8_t xqs[512];
            float v = 0.f;
            for (int w = 0; w < 16; ++w) {
                for (int l = 0; l < 32; ++l) sq[l] = Rp[col0 + 32 * w + l] * Rp[col0 + 32 * w + l];
                v += butterfly_sum(sq, 32);
            }
            ssp[s] = v;
            for (int j = 0; j < 512; ++j) xs[j] = Rp[col0 + j] * w_norm[col0 + j];
            for (int b = 0; b < 16; ++b) q8_block_f(xs + 32 * b, xqs + 32 * b, &xd[b]);
            for (int row = 0; row < ROWS; ++row) {
                if (row >= LR && !w_inj) {
                    part[(size_t) s * ROWS + row] = 0.f;
                    continue;
                }
                float acc[8];
                for (int j = 0; j < 8; ++j) {
                    float a = 0.f;
                    for (int q = 0; q < 8; ++q) {
                        const int ch = q * 8 + j;
                        if (row < LR) {
                            const int8_t* w = dq + (size_t) row * D + col0 + ch * 8;
                            int dot = 0;
                            for (int m = 0; m < 8; ++m) dot += (int) w[m] * (int) xqs[ch * 8 + m];
                            const float wsc = orc_f16_to_f32(dd[((size_t) row * D + col0) / 32 + ch / 4]);
                            a = fmaf(wsc * xd[ch / 4], (float) dot, a);
                        } else {
                            const uint16_t* h = w_inj + (size_t) (row - LR) * D + col0 + ch * 8;
                            float e = bf16_f(h[0]) * xs[ch * 8];
                            for (int m = 1; m < 8; ++m) e = e + bf16_f(h[m]) * xs[ch * 8 + m];
                            a = a + e;
                        }
                    }
                    acc[j] = a;
                }
                part[(size_t) s * ROWS + row] = butterfly_up(acc, 8);
            }
        }
        if (part_out) memcpy(part_out + (size_t) t * NS * ROWS, part, (size_t) NS * ROWS * sizeof(float));
        if (ssp_out) memcpy(ssp_out + (size_t) t * NS, ssp, (size_t) NS * sizeof(float));
        for (int c = 0; c < HC; ++c) {
            float v = 0.f;
            for (int ss = 0; ss < SPS; ++ss) v += ssp[c * SPS + ss];
            rs[c] = 1.0f / sqrtf(v / (float) N + eps);
        }
        for (int r = 0; r < ROWS; ++r) {
            if (r >= LR && !w_inj) break;
            float sum = 0.f;
            for (int c = 0; c < HC; ++c) {
                float p = 0.f;
                for (int ss = 0; ss < SPS; ++ss) p += part[(size_t) (c * SPS + ss) * ROWS + r];
                sum = fmaf(rs[c], p, sum);
            }
            if (r < LR) lo[r] = silu_(sum / (float) HC);
            else if (inject) inject[t * HC + (r - LR)] = sum;
        }
        for (int b = 0; b < LR / 32; ++b) q8_block_f(lo + 32 * b, loq + 32 * b, &lod[b]);
        for (int i = 0; i < N; ++i) {
            for (int c = 0; c < HC; ++c) {
                const size_t u = (size_t) c * N + i;
                float v16[16];
                for (int L = 0; L < 16; ++L) {
                    if (L >= LR / 32) {
                        v16[L] = 0.f;
                        continue;
                    }
                    int dot = 0;
                    for (int m = 0; m < 32; ++m) dot += (int) uq[u * LR + 32 * L + m] * (int) loq[32 * L + m];
                    v16[L] = orc_f16_to_f32(ud[u * (LR / 32) + L]) * lod[L] * (float) dot;
                }
                const float g = butterfly_up(v16, 16);
                gs[c] = sigm_(g) * (Rp[u] * w_norm[u] * rs[c]);
            }
            float m = gs[0];
            for (int c = 1; c < HC; ++c) m += gs[c];
            mixed[(size_t) t * N + i] = m / (float) HC;
        }
        if (xq) orc_quantize_q8_1(mixed + (size_t) t * N, xq + (size_t) t * (N / 32) * ORC_Q81_BYTES, N, 1);
        if (bo) memcpy(R + (size_t) t * D, Rp, (size_t) D * sizeof(float));
    }
    free(Rp);
    free(part);
    free(ssp);
    free(lo);
    free(loq);
}
