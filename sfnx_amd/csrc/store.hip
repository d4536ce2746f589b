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

// one Q4_K super-block per thread: per 32-value sub-block min' = min(0, min x) and scale = (max - min') / 15, d and
// dmin the largest of each over 63 as f16, 6-bit sc and m against the stored f16, 4-bit q = round((x + dmin m) / (d sc))
__global__ void k_quant_q4k(const float* __restrict__ x, uint8_t* __restrict__ dst, int64_t nblk) {
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x;
    if (k >= nblk) return;
    const float* v = x + k * 256;
    uint8_t* b = dst + k * Q4K_BYTES;
    float scale[8], mn8[8], max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; ++j) {
        float mn = v[32 * j], mx = v[32 * j];
        for (int l = 1; l < 32; ++l) {
            const float t = v[32 * j + l];
            if (t < mn) mn = t;
            if (t > mx) mx = t;
        }
        if (mn > 0.f) mn = 0.f;
        scale[j] = (mx - mn) / 15.0f;
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
    for (int jp = 0; jp < 4; ++jp) {
        const int j0 = 2 * jp, j1 = j0 + 1;
        const float dl0 = df * (float) sc[j0], ml0 = mf * (float) m[j0];
        const float dl1 = df * (float) sc[j1], ml1 = mf * (float) m[j1];
        for (int l = 0; l < 32; ++l) {
            const int q0 = dl0 > 0.f ? clampi((int) roundf((v[32 * j0 + l] + ml0) / dl0), 0, 15) : 0;
            const int q1 = dl1 > 0.f ? clampi((int) roundf((v[32 * j1 + l] + ml1) / dl1), 0, 15) : 0;
            b[16 + 32 * jp + l] = (uint8_t) (q0 | (q1 << 4));
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

// ------------------------------------------------------------------------------------------------ packing
// Q4_K: thread per (row, super-block).  Nibble bytes 32 jg + 16 h + x of super-block b land in the row's run b / 2 at
// 128 h + 16 ((b % 2) 4 + jg) + x; the 16 header bytes at the header plane's (row, b).
template <bool PACK>
__global__ void k_pack_q4k(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t n_mat, int R, int C) {
    const int nb = C / 256;
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x, per_mat = (int64_t) R * nb;
    if (k >= n_mat * per_mat) return;
    const int64_t m = k / per_mat;
    const int r = (int) ((k % per_mat) / nb), b = (int) (k % nb);
    const size_t mat_bytes = (size_t) R * nb * Q4K_BYTES;
    const size_t gg = m * mat_bytes + ((size_t) r * nb + b) * Q4K_BYTES;                          // GGUF block
    const Q4kPlanes P = q4k_planes((const uint8_t*) nullptr + m * mat_bytes, R, C);
    const size_t hdr = (size_t) P.hdr16(r, C, b);
    for (int i = 0; i < 16; ++i) {
        if (PACK) dst[hdr + i] = src[gg + i];
        else dst[gg + i] = src[hdr + i];
    }
    for (int jg = 0; jg < 4; ++jg)
        for (int h = 0; h < 2; ++h)
            for (int x = 0; x < 16; ++x) {
                // the run's byte 128 h + 16 ((b % 2) 4 + jg) + x
                const size_t pg = gg + 16 + 32 * jg + 16 * h + x,
                             pp = (size_t) P.nib16(r, C, 16 * (b / 2) + 8 * h + (b % 2) * 4 + jg) + x;
                if (PACK) dst[pp] = src[pg];
                else dst[pg] = src[pp];
            }
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

// ------------------------------------------------------------------------------------------------ dequant
// thread per (row, 32-value sub-block) of the planar store; F16: the tensor-core path's f16 weight
template <bool F16>
__global__ void k_deq_q4k(const uint8_t* __restrict__ src, void* __restrict__ out, int64_t n_mat, int R, int C) {
    const int ns = C / 32;
    const int64_t k = blockIdx.x * (int64_t) blockDim.x + threadIdx.x, per_mat = (int64_t) R * ns;
    if (k >= n_mat * per_mat) return;
    const int64_t m = k / per_mat;
    const int r = (int) ((k % per_mat) / ns), s = (int) (k % ns), b = s / 8, j = s % 8, jg = j / 2, hi = j % 2;
    const Q4kPlanes P = q4k_planes(src + m * ((size_t) R * (C / 256) * Q4K_BYTES), R, C);
    const uint4 h = *reinterpret_cast<const uint4*>(P.hdr16(r, C, b));
    const float d = h2f((uint16_t) (h.x & 0xffff)), dmin = h2f((uint16_t) (h.x >> 16));
    float sc, mm;
    q4k_scale_min(h, j, sc, mm);
    // the run's pieces 4 (b % 2) + jg (values 0-15) and 8 + 4 (b % 2) + jg (values 16-31)
    const int p0 = 16 * (b / 2) + (b % 2) * 4 + jg;
    const size_t o = (size_t) m * R * C + (size_t) r * C + 32 * s;
    if (F16) {
        const __half d1 = __float2half_rn(d * sc), nm1 = __float2half_rn(-(dmin * mm));
        for (int l = 0; l < 32; ++l) {
            const int q = (P.nib16(r, C, p0 + 8 * (l / 16))[l % 16] >> (4 * hi)) & 0xF;
            ((__half*) out)[o + l] = __hfma(__int2half_rn(q), d1, nm1);
        }
    } else {
        const float d1 = d * sc, m1 = dmin * mm;
        for (int l = 0; l < 32; ++l) {
            const int q = (P.nib16(r, C, p0 + 8 * (l / 16))[l % 16] >> (4 * hi)) & 0xF;
            ((float*) out)[o + l] = d1 * (float) q - m1;
        }
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

inline unsigned blocks_for(int64_t n, int t) { return (unsigned) ((n + t - 1) / t); }
void check_type_shape(uint32_t type, int rows, int cols) {
    require(type == SFNX_Q4_K || type == SFNX_Q8_0, "weight type must be Q4_K (12) or Q8_0 (8)");
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
        require(type == SFNX_Q4_K || type == SFNX_Q8_0, "weight type must be Q4_K (12) or Q8_0 (8)");
        require(cols > 0 && cols % (type == SFNX_Q4_K ? 256 : 32) == 0, "columns must be whole blocks");
        if (rows <= 0) return;
        if (type == SFNX_Q4_K) {
            const int64_t nb = rows * (cols / 256);
            k_quant_q4k<<<blocks_for(nb, 128), 128, 0, stream_of(st)>>>(x, (uint8_t*) gguf, nb);
        } else {
            const int64_t nb = rows * (cols / 32);
            k_quant_q80<<<blocks_for(nb, 256), 256, 0, stream_of(st)>>>(x, (uint8_t*) gguf, nb);
        }
    });
}

extern "C" int sfnx_store_pack(uint32_t type, const void* gguf, void* planar, int64_t n_mat, int R, int C, void* st) {
    return guarded("sfnx_store_pack", [&] {
        check_type_shape(type, R, C);
        require(gguf != planar, "packing is out of place");
        const int64_t n = n_mat * R * (type == SFNX_Q4_K ? C / 256 : C / 32);
        if (n <= 0) return;
        if (type == SFNX_Q4_K)
            k_pack_q4k<true><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>((const uint8_t*) gguf, (uint8_t*) planar, n_mat, R, C);
        else
            k_pack_q80<true><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>((const uint8_t*) gguf, (uint8_t*) planar, n_mat, R, C);
    });
}

extern "C" int sfnx_store_unpack(uint32_t type, const void* planar, void* gguf, int64_t n_mat, int R, int C, void* st) {
    return guarded("sfnx_store_unpack", [&] {
        check_type_shape(type, R, C);
        require(gguf != planar, "unpacking is out of place");
        const int64_t n = n_mat * R * (type == SFNX_Q4_K ? C / 256 : C / 32);
        if (n <= 0) return;
        if (type == SFNX_Q4_K)
            k_pack_q4k<false><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>((const uint8_t*) planar, (uint8_t*) gguf, n_mat, R, C);
        else
            k_pack_q80<false><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>((const uint8_t*) planar, (uint8_t*) gguf, n_mat, R, C);
    });
}

extern "C" int sfnx_dequantize(uint32_t type, const void* planar, float* y, int64_t n_mat, int R, int C, void* st) {
    return guarded("sfnx_dequantize", [&] {
        check_type_shape(type, R, C);
        const int64_t n = n_mat * R * (C / 32);
        if (n <= 0) return;
        if (type == SFNX_Q4_K) k_deq_q4k<false><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>((const uint8_t*) planar, y, n_mat, R, C);
        else k_deq_q80<false><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>((const uint8_t*) planar, y, n_mat, R, C);
    });
}

extern "C" int sfnx_dequantize_f16(uint32_t type, const void* planar, uint16_t* y, int64_t n_mat, int R, int C, void* st) {
    return guarded("sfnx_dequantize_f16", [&] {
        check_type_shape(type, R, C);
        const int64_t n = n_mat * R * (C / 32);
        if (n <= 0) return;
        if (type == SFNX_Q4_K) k_deq_q4k<true><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>((const uint8_t*) planar, y, n_mat, R, C);
        else k_deq_q80<true><<<blocks_for(n, 256), 256, 0, stream_of(st)>>>((const uint8_t*) planar, y, n_mat, R, C);
    });
}
