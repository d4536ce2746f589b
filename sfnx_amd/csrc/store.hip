// The expert-weight store: seeded synthetic values, the Q4_K / Q8_0 quantizers, GGUF <-> planar packing and
// dequantization.  One-time work (loading or generating a model), so the kernels favour plainness over speed.
#include "common.hpp"

namespace sfnx {

static thread_local std::string g_err;
void set_error(const std::string& msg) { g_err = msg; }

namespace {

// ------------------------------------------------------------------------------------------------ synthetic values
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
// Irwin-Hall(12): the sum of twelve 24-bit uniforms minus 6, an integer until the one conversion to float
__global__ void k_synth(float* out, size_t n, uint64_t seed, uint64_t offset, float stdv) {
    for (size_t i = blockIdx.x * (size_t) blockDim.x + threadIdx.x; i < n; i += (size_t) gridDim.x * blockDim.x) {
        const uint64_t c = offset + i;
        int64_t s = 0;
#pragma unroll
        for (int m = 0; m < 6; ++m) {
            const uint64_t r = mix64(seed + (6 * c + (uint64_t) m + 1) * 0x9e3779b97f4a7c15ull);
            s += (int64_t) (r & 0xffffffu) + (int64_t) ((r >> 32) & 0xffffffu);
        }
        const float z = (float) (int32_t) (s - 6 * (1ll << 24)) * 5.9604644775390625e-8f;
        out[i] = z * stdv;
    }
}

// ------------------------------------------------------------------------------------------------ quantizers
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

// one K-quant super-block per thread, Q4_K (Q5 false: 15 levels) or Q5_K (31 levels, the fifth bit in qh): per
// 32-value sub-block min' = min(0, min x) and scale = (max - min') / levels, d and dmin the largest of each over 63 as
// f16, 6-bit sc and m against the stored f16, q = round((x + dmin m) / (d sc))
template <bool Q5>
__global__ void k_quant_kq(const float* __restrict__ x, uint8_t* __restrict__ dst, int64_t nblk) {
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x;
    if (k >= nblk) return;
    const float levels = Q5 ? 31.0f : 15.0f;
    const int qmax = Q5 ? 31 : 15;
    const float* v = x + k * 256;
    uint8_t* b = dst + k * (Q5 ? Q5K_BYTES : Q4K_BYTES);
    float scale[8], mn8[8], max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; ++j) {
        float mn = v[32 * j], mx = v[32 * j];
        for (int l = 1; l < 32; ++l) {
            const float t = v[32 * j + l];
            if (t < mn) mn = t;
            if (t > mx) mx = t;
        }
        if (mn > 0.f) mn = 0.f;
        scale[j] = (mx - mn) / levels;
        mn8[j] = mn < 0.f ? -mn : 0.f;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (mn8[j] > max_min) max_min = mn8[j];
    }
    const uint16_t dh = f2h(max_scale / 63.0f), mh = f2h(max_min / 63.0f);
    const float df = h2f(dh), mf = h2f(mh);
    int sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = df > 0.f ? clampi((int) roundf(scale[j] / df), 0, 63) : 0;
        m[j] = mf > 0.f ? clampi((int) roundf(mn8[j] / mf), 0, 63) : 0;
    }
    b[0] = dh & 0xff;
    b[1] = dh >> 8;
    b[2] = mh & 0xff;
    b[3] = mh >> 8;
    for (int j = 0; j < 4; ++j) {
        b[4 + j] = (uint8_t) ((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        b[8 + j] = (uint8_t) ((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        b[12 + j] = (uint8_t) ((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t* qh = b + 16;
    uint8_t* qs = b + (Q5 ? 48 : 16);
    for (int jp = 0; jp < 4; ++jp) {
        const int j0 = 2 * jp, j1 = j0 + 1;
        const float dl0 = df * (float) sc[j0], ml0 = mf * (float) m[j0];
        const float dl1 = df * (float) sc[j1], ml1 = mf * (float) m[j1];
        for (int l = 0; l < 32; ++l) {
            const int q0 = dl0 > 0.f ? clampi((int) roundf((v[32 * j0 + l] + ml0) / dl0), 0, qmax) : 0;
            const int q1 = dl1 > 0.f ? clampi((int) roundf((v[32 * j1 + l] + ml1) / dl1), 0, qmax) : 0;
            qs[32 * jp + l] = (uint8_t) ((q0 & 15) | ((q1 & 15) << 4));
            if (Q5) qh[l] = (uint8_t) ((jp ? qh[l] : 0) | ((q0 >> 4) << j0) | ((q1 >> 4) << j1));
        }
    }
}

// one Q8_0 block per thread, tools/mtp_experts.py:44-55: d = amax / 127, q = sign(v) floor(|v| + 0.5), v = x (1 / d)
__global__ void k_quant_q80(const float* __restrict__ x, uint8_t* __restrict__ dst, int64_t nblk) {
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x;
    if (k >= nblk) return;
    const float* v = x + k * 32;
    uint8_t* b = dst + k * Q80_BYTES;
    float amax = 0.f;
    for (int l = 0; l < 32; ++l) amax = fabsf(v[l]) > amax ? fabsf(v[l]) : amax;
    const float d = amax / 127.0f, idv = d != 0.f ? 1.0f / d : 0.f;
    const uint16_t dh = f2h(d);
    b[0] = dh & 0xff;
    b[1] = dh >> 8;
    for (int l = 0; l < 32; ++l) {
        const float t = v[l] * idv;
        const float a = floorf(fabsf(t) + 0.5f);
        b[2 + l] = (uint8_t) (int8_t) (int) (t < 0.f ? -a : a);
    }
}

// one Q4_0 block per thread, tools/mtp_experts.py:29-41: d = (the first value of largest magnitude) / -8,
// q = min(15, trunc(x (1 / d) + 8.5))
__global__ void k_quant_q40(const float* __restrict__ x, uint8_t* __restrict__ dst, int64_t nblk) {
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x;
    if (k >= nblk) return;
    const float* v = x + k * 32;
    uint8_t* b = dst + k * Q40_BYTES;
    float amax = fabsf(v[0]), mx = v[0];   // the first value of largest magnitude (numpy's argmax)
    for (int l = 1; l < 32; ++l)
        if (fabsf(v[l]) > amax) {
            amax = fabsf(v[l]);
            mx = v[l];
        }
    const float d = mx / -8.0f, idv = d != 0.f ? 1.0f / d : 0.f;
    // d = mx / -8 is exact; a zero d keeps the opposite of mx's sign (the compiler's fused f32 -> f16 conversion of the
    // product would give +0 for -0)
    const uint16_t dh = mx == 0.f ? (uint16_t) (((__float_as_uint(mx) >> 16) & 0x8000u) ^ 0x8000u) : f2h(d);
    b[0] = dh & 0xff;
    b[1] = dh >> 8;
    for (int l = 0; l < 16; ++l) {
        const float a = truncf(v[l] * idv + 8.5f), c = truncf(v[l + 16] * idv + 8.5f);
        const int q0 = (int) (a < 15.f ? a : 15.f), q1 = (int) (c < 15.f ? c : 15.f);
        b[2 + l] = (uint8_t) (q0 | (q1 << 4));
    }
}

// one Q5_1 block per thread, ggml's closed form: m = min, d = (max - min) / 31, q = trunc((x - m) (1 / d) + 0.5)
__global__ void k_quant_q51(const float* __restrict__ x, uint8_t* __restrict__ dst, int64_t nblk) {
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x;
    if (k >= nblk) return;
    const float* v = x + k * 32;
    uint8_t* b = dst + k * Q51_BYTES;
    float mn = v[0], mx = v[0];
    for (int l = 1; l < 32; ++l) {
        if (v[l] < mn) mn = v[l];
        if (v[l] > mx) mx = v[l];
    }
    const float d = (mx - mn) / 31.0f, idv = d != 0.f ? 1.0f / d : 0.f;
    const uint16_t dh = f2h(d), mh = f2h(mn);
    b[0] = dh & 0xff;
    b[1] = dh >> 8;
    b[2] = mh & 0xff;
    b[3] = mh >> 8;
    uint32_t qh = 0;
    for (int l = 0; l < 16; ++l) {
        const int q0 = (int) truncf((v[l] - mn) * idv + 0.5f), q1 = (int) truncf((v[l + 16] - mn) * idv + 0.5f);
        b[8 + l] = (uint8_t) ((q0 & 15) | ((q1 & 15) << 4));
        qh |= (uint32_t) ((q0 >> 4) & 1) << l;
        qh |= (uint32_t) ((q1 >> 4) & 1) << (l + 16);
    }
    for (int i = 0; i < 4; ++i) b[4 + i] = (uint8_t) (qh >> (8 * i));
}

// ------------------------------------------------------------------------------------------------ packing
// K-quants: thread per (row, super-block).  Nibble bytes 32 jg + 16 h + x of super-block b land in piece
// 16 (b / 2) + 8 h + 4 (b % 2) + jg of the row's nibbles (the run b / 2 in [half][group] order), byte x; the 16 header
// bytes are header piece b; Q5_K's qh bytes 16 h + x are qh piece 2 b + h.
template <bool Q5, bool PACK>
__global__ void k_pack_kq(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t n_mat, int R, int C) {
    constexpr int BB = Q5 ? Q5K_BYTES : Q4K_BYTES, QS = Q5 ? 48 : 16;
    const int nb = C / 256;
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x, per_mat = (int64_t) R * nb;
    if (k >= n_mat * per_mat) return;
    const int64_t m = k / per_mat;
    const int r = (int) ((k % per_mat) / nb), b = (int) (k % nb);
    const size_t mat_bytes = (size_t) R * nb * BB;
    const size_t gg = m * mat_bytes + ((size_t) r * nb + b) * BB;   // GGUF block
    const KqPlanes P = kq_planes<Q5>((const uint8_t*) nullptr + m * mat_bytes, R, C);
    auto mv = [&](size_t pg, size_t pp) {
        if (PACK) dst[pp] = src[pg];
        else dst[pg] = src[pp];
    };
    for (int i = 0; i < 16; ++i) mv(gg + i, (size_t) P.hdr16(r, C, b) + i);
    if (Q5)
        for (int i = 0; i < 32; ++i) mv(gg + 16 + i, (size_t) P.qh16(r, C, 2 * b + i / 16) + i % 16);
    for (int jg = 0; jg < 4; ++jg)
        for (int h = 0; h < 2; ++h)
            for (int x = 0; x < 16; ++x)
                mv(gg + QS + 32 * jg + 16 * h + x, (size_t) P.nib16(r, C, 16 * (b / 2) + 8 * h + (b % 2) * 4 + jg) + x);
}
// Q8_0: thread per (row, block).  Quant bytes 16 h + x of block b land in the row's 512-byte run b / 16 at
// 256 h + 16 (b % 16) + x; the scale at the scale plane's (row, b).
template <bool PACK>
__global__ void k_pack_q80(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t n_mat, int R, int C) {
    const int nb = C / 32;
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x, per_mat = (int64_t) R * nb;
    if (k >= n_mat * per_mat) return;
    const int64_t m = k / per_mat;
    const int r = (int) ((k % per_mat) / nb), b = (int) (k % nb);
    const size_t mat_bytes = (size_t) R * nb * Q80_BYTES;
    const size_t gg = m * mat_bytes + ((size_t) r * nb + b) * Q80_BYTES;
    const Q80Planes P = q80_planes((const uint8_t*) nullptr + m * mat_bytes, R, C);
    const size_t dp = (size_t) P.dof(r, C, b);
    for (int i = 0; i < 2; ++i) {
        if (PACK) dst[dp + i] = src[gg + i];
        else dst[gg + i] = src[dp + i];
    }
    for (int h = 0; h < 2; ++h)
        for (int x = 0; x < 16; ++x) {
            // the run's byte 256 h + 16 (b % 16) + x
            const size_t pg = gg + 2 + 16 * h + x, pp = (size_t) P.q16(r, C, 32 * (b / 16) + 16 * h + b % 16) + x;
            if (PACK) dst[pp] = src[pg];
            else dst[pg] = src[pp];
        }
}

// Q4_0 / Q5_1: thread per (row, block).  The 16 quant bytes are piece b of the row's nibbles; Q4_0's d is at the d
// plane's (row, b), Q5_1's (d, m) and qh words at those planes' (row, b).
template <int TYPE, bool PACK>
__global__ void k_pack_nb(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t n_mat, int R, int C) {
    constexpr int BB = TYPE == SFNX_Q4_0 ? Q40_BYTES : Q51_BYTES, QS = TYPE == SFNX_Q4_0 ? 2 : 8;
    const int nb = C / 32;
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x, per_mat = (int64_t) R * nb;
    if (k >= n_mat * per_mat) return;
    const int64_t m = k / per_mat;
    const int r = (int) ((k % per_mat) / nb), b = (int) (k % nb);
    const size_t mat_bytes = (size_t) R * nb * BB;
    const size_t gg = m * mat_bytes + ((size_t) r * nb + b) * BB;
    const NbPlanes P = nb_planes<TYPE>((const uint8_t*) nullptr + m * mat_bytes, R, C);
    auto mv = [&](size_t pg, size_t pp) {
        if (PACK) dst[pp] = src[pg];
        else dst[pg] = src[pp];
    };
    if (TYPE == SFNX_Q4_0) {
        for (int i = 0; i < 2; ++i) mv(gg + i, (size_t) P.d_of(r, C, b) + i);
    } else {
        for (int i = 0; i < 4; ++i) mv(gg + i, (size_t) P.dm_of(r, C, b) + i);
        for (int i = 0; i < 4; ++i) mv(gg + 4 + i, (size_t) P.qh_of(r, C, b) + i);
    }
    for (int i = 0; i < 16; ++i) mv(gg + QS + i, (size_t) P.q16(r, C, b) + i);
}

// ------------------------------------------------------------------------------------------------ dequant
// thread per (row, 32-value sub-block) of the planar store; F16: the tensor-core path's f16 weight
template <bool Q5, bool F16>
__global__ void k_deq_kq(const uint8_t* __restrict__ src, void* __restrict__ out, int64_t n_mat, int R, int C) {
    const int ns = C / 32;
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x, per_mat = (int64_t) R * ns;
    if (k >= n_mat * per_mat) return;
    const int64_t m = k / per_mat;
    const int r = (int) ((k % per_mat) / ns), s = (int) (k % ns), b = s / 8, j = s % 8, jg = j / 2, hi = j % 2;
    const KqPlanes P = kq_planes<Q5>(src + m * ((size_t) R * (C / 256) * (Q5 ? Q5K_BYTES : Q4K_BYTES)), R, C);
    const uint4 h = *reinterpret_cast<const uint4*>(P.hdr16(r, C, b));
    const float d = h2f((uint16_t) (h.x & 0xffff)), dmin = h2f((uint16_t) (h.x >> 16));
    float sc, mm;
    q4k_scale_min(h, j, sc, mm);
    // the run's pieces 4 (b % 2) + jg (values 0-15) and 8 + 4 (b % 2) + jg (values 16-31)
    const int p0 = 16 * (b / 2) + (b % 2) * 4 + jg;
    auto value = [&](int l) {
        const int nib = (P.nib16(r, C, p0 + 8 * (l / 16))[l % 16] >> (4 * hi)) & 0xF;
        return Q5 ? nib | (((P.qh16(r, C, 2 * b + l / 16)[l % 16] >> j) & 1) << 4) : nib;
    };
    const size_t o = (size_t) m * R * C + (size_t) r * C + 32 * s;
    if (F16) {
        const __half d1 = __float2half_rn(d * sc), nm1 = __float2half_rn(-(dmin * mm));
        for (int l = 0; l < 32; ++l) ((__half*) out)[o + l] = __hfma(__int2half_rn(value(l)), d1, nm1);
    } else {
        const float d1 = d * sc, m1 = dmin * mm;
        for (int l = 0; l < 32; ++l) ((float*) out)[o + l] = d1 * (float) value(l) - m1;
    }
}
template <bool F16>
__global__ void k_deq_q80(const uint8_t* __restrict__ src, void* __restrict__ out, int64_t n_mat, int R, int C) {
    const int nb = C / 32;
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x, per_mat = (int64_t) R * nb;
    if (k >= n_mat * per_mat) return;
    const int64_t m = k / per_mat;
    const int r = (int) ((k % per_mat) / nb), b = (int) (k % nb);
    const Q80Planes P = q80_planes(src + m * ((size_t) R * nb * Q80_BYTES), R, C);
    const uint16_t dh = *P.dof(r, C, b);
    const int p0 = 32 * (b / 16) + b % 16;   // the block's first half; the second 16 pieces on
    const size_t o = (size_t) m * R * C + (size_t) r * C + 32 * b;
    for (int l = 0; l < 32; ++l) {
        const int v = (int8_t) P.q16(r, C, p0 + 16 * (l / 16))[l % 16];
        if (F16) ((__half*) out)[o + l] = __hmul(__int2half_rn(v), __ushort_as_half(dh));
        else ((float*) out)[o + l] = h2f(dh) * (float) v;
    }
}

// Q4_0 / Q5_1: thread per (row, block); F16: the tensor-core path's weight (Q4_0 hmul2(q - 8, d), Q5_1 hfma2(q, d, m))
template <int TYPE, bool F16>
__global__ void k_deq_nb(const uint8_t* __restrict__ src, void* __restrict__ out, int64_t n_mat, int R, int C) {
    const int nb = C / 32;
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x, per_mat = (int64_t) R * nb;
    if (k >= n_mat * per_mat) return;
    const int64_t m = k / per_mat;
    const int r = (int) ((k % per_mat) / nb), b = (int) (k % nb);
    const NbPlanes P = nb_planes<TYPE>(src + m * row_bytes(TYPE, C) * R, R, C);
    const uint8_t* q = P.q16(r, C, b);
    uint16_t dh, mh = 0;
    uint32_t qh = 0;
    if (TYPE == SFNX_Q4_0) {
        dh = *reinterpret_cast<const uint16_t*>(P.d_of(r, C, b));
    } else {
        const uint32_t dm = *reinterpret_cast<const uint32_t*>(P.dm_of(r, C, b));
        dh = (uint16_t) (dm & 0xffff);
        mh = (uint16_t) (dm >> 16);
        qh = *reinterpret_cast<const uint32_t*>(P.qh_of(r, C, b));
    }
    const size_t o = (size_t) m * R * C + (size_t) r * C + 32 * b;
    for (int l = 0; l < 32; ++l) {
        const int nib = l < 16 ? q[l] & 15 : q[l - 16] >> 4;
        const int v = TYPE == SFNX_Q4_0 ? nib - 8 : nib | (int) (((qh >> l) & 1) << 4);
        if (F16) {
            const __half d = __ushort_as_half(dh);
            ((__half*) out)[o + l] = TYPE == SFNX_Q4_0 ? __hmul(__int2half_rn(v), d) : __hfma(__int2half_rn(v), d, __ushort_as_half(mh));
        } else {
            ((float*) out)[o + l] = TYPE == SFNX_Q4_0 ? (float) v * h2f(dh) : h2f(dh) * (float) v + h2f(mh);
        }
    }
}

inline unsigned blocks_for(int64_t n, int t) { return (unsigned) ((n + t - 1) / t); }
void check_type_shape(uint32_t type, int rows, int cols) {
    require(expert_type_ok(type), "weight type must be Q4_0 (2), Q5_1 (7), Q8_0 (8), Q4_K (12) or Q5_K (13)");
    require(cols > 0 && cols % 512 == 0, "columns must be a positive multiple of 512");
    require(rows >= 0 && rows % ROWTILE == 0, "rows must be a multiple of 32 (the store's row tile)");
}

}  // namespace
}  // namespace sfnx

using namespace sfnx;

extern "C" const char* sfnx_last_error(void) { return g_err.c_str(); }
extern "C" int sfnx_abi_version(void) { return 1; }
extern "C" size_t sfnx_row_bytes(uint32_t type, int cols) { return row_bytes(type, cols); }

extern "C" int sfnx_synth_normal(float* out, size_t n, uint64_t seed, uint64_t offset, float stdv, void* st) {
    return guarded("sfnx_synth_normal", [&] {
        if (!n) return;
        k_synth<<<(unsigned) std::min<size_t>((n + 255) / 256, 65536), 256, 0, stream_of(st)>>>(out, n, seed, offset, stdv);
    });
}

extern "C" int sfnx_quantize_weights(uint32_t type, const float* x, void* gguf, int64_t rows, int cols, void* st) {
    return guarded("sfnx_quantize_weights", [&] {
        require(expert_type_ok(type), "weight type must be Q4_0 (2), Q5_1 (7), Q8_0 (8), Q4_K (12) or Q5_K (13)");
        require(cols > 0 && cols % block_values(type) == 0, "columns must be whole blocks");
        if (rows <= 0) return;
        const int64_t nb = rows * (cols / block_values(type));
        if (type == SFNX_Q4_K) k_quant_kq<false><<<blocks_for(nb, 128), 128, 0, stream_of(st)>>>(x, (uint8_t*) gguf, nb);
        else if (type == SFNX_Q5_K) k_quant_kq<true><<<blocks_for(nb, 128), 128, 0, stream_of(st)>>>(x, (uint8_t*) gguf, nb);
        else if (type == SFNX_Q4_0) k_quant_q40<<<blocks_for(nb, 256), 256, 0, stream_of(st)>>>(x, (uint8_t*) gguf, nb);
        else if (type == SFNX_Q5_1) k_quant_q51<<<blocks_for(nb, 256), 256, 0, stream_of(st)>>>(x, (uint8_t*) gguf, nb);
        else k_quant_q80<<<blocks_for(nb, 256), 256, 0, stream_of(st)>>>(x, (uint8_t*) gguf, nb);
    });
}

namespace {
template <bool PACK> void pack(uint32_t type, const void* src, void* dst, int64_t n_mat, int R, int C, void* st) {
    check_type_shape(type, R, C);
    require(src != dst, "packing is out of place");
    const int64_t n = n_mat * R * (C / block_values(type));
    if (n <= 0) return;
    const auto* s8 = (const uint8_t*) src;
    auto* d8 = (uint8_t*) dst;
    if (type == SFNX_Q4_K) k_pack_kq<false, PACK><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>(s8, d8, n_mat, R, C);
    else if (type == SFNX_Q5_K) k_pack_kq<true, PACK><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>(s8, d8, n_mat, R, C);
    else if (type == SFNX_Q4_0) k_pack_nb<SFNX_Q4_0, PACK><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>(s8, d8, n_mat, R, C);
    else if (type == SFNX_Q5_1) k_pack_nb<SFNX_Q5_1, PACK><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>(s8, d8, n_mat, R, C);
    else k_pack_q80<PACK><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>(s8, d8, n_mat, R, C);
}
template <bool F16> void dequant(uint32_t type, const void* planar, void* y, int64_t n_mat, int R, int C, void* st) {
    check_type_shape(type, R, C);
    const int64_t n = n_mat * R * (C / 32);
    if (n <= 0) return;
    const auto* p = (const uint8_t*) planar;
    if (type == SFNX_Q4_K) k_deq_kq<false, F16><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>(p, y, n_mat, R, C);
    else if (type == SFNX_Q5_K) k_deq_kq<true, F16><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>(p, y, n_mat, R, C);
    else if (type == SFNX_Q4_0) k_deq_nb<SFNX_Q4_0, F16><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>(p, y, n_mat, R, C);
    else if (type == SFNX_Q5_1) k_deq_nb<SFNX_Q5_1, F16><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>(p, y, n_mat, R, C);
    else k_deq_q80<F16><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>(p, y, n_mat, R, C);
}
}  // namespace

extern "C" int sfnx_store_pack(uint32_t type, const void* gguf, void* planar, int64_t n_mat, int R, int C, void* st) {
    return guarded("sfnx_store_pack", [&] { pack<true>(type, gguf, planar, n_mat, R, C, st); });
}

extern "C" int sfnx_store_unpack(uint32_t type, const void* planar, void* gguf, int64_t n_mat, int R, int C, void* st) {
    return guarded("sfnx_store_unpack", [&] { pack<false>(type, planar, gguf, n_mat, R, C, st); });
}

extern "C" int sfnx_dequantize(uint32_t type, const void* planar, float* y, int64_t n_mat, int R, int C, void* st) {
    return guarded("sfnx_dequantize", [&] { dequant<false>(type, planar, y, n_mat, R, C, st); });
}

extern "C" int sfnx_dequantize_f16(uint32_t type, const void* planar, uint16_t* y, int64_t n_mat, int R, int C, void* st) {
    return guarded("sfnx_dequantize_f16", [&] { dequant<true>(type, planar, y, n_mat, R, C, st); });
}
