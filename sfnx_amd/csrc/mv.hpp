// Device building blocks of the expert kernels: jobs and activations in LDS, and a lane group's share of one Q4_K,
// Q5_K or Q8_0 weight row dotted with int8 activations (v_dot4_i32_i8).  The arithmetic per (row, activation row):
//   Q4_K: 8 lanes a row, lane l8 the 64-value groups l8 + 8 i in order (src/moe_q4k.cuh:30-86), each group
//         d (d8l (sc0 dl) + d8h (sc1 dh)) - dmin (d8l (m0 sl) + d8h (m1 sh)), then xor 4, 2, 1 (src/moe.cuh:224-235).
//   Q5_K: the same on the 5-bit values (the fifth bit of value l of sub-block j is bit j of qh[l]).
//   Q8_0: 16 lanes a row, lane l16 the 32-blocks l16 + 16 i in order, each (d_w d_a) sum(q_w q_a), then xor 8 .. 1.
#pragma once
#include "common.hpp"

namespace sfnx {



// a job into LDS (BigJob or Job)
template <typename J> __device__ __forceinline__ void load_job(J& jb, const J* src) {
    for (int k = threadIdx.x; k < (int) (sizeof(J) / 4); k += blockDim.x) reinterpret_cast<int*>(&jb)[k] = reinterpret_cast<const int*>(src)[k];
}

// LDS activations for up to TT rows of K values: int8 values, the f16-rounded block scale as float, the block's sum
struct Acts {
    int8_t* q;
    float* d;
    int* s;
    int K;
    __device__ __forceinline__ const int4* q4(int j, int blk) const { return reinterpret_cast<const int4*>(q + (size_t) j * K + 32 * blk); }
};
__device__ __forceinline__ Acts acts_in(unsigned char* lds, int TT, int K) {
    Acts a;
    a.q = reinterpret_cast<int8_t*>(lds);
    a.d = reinterpret_cast<float*>(lds + (size_t) TT * K);
    a.s = reinterpret_cast<int*>(lds + (size_t) TT * K + (size_t) TT * (K / 32) * 4);
    a.K = K;
    return a;
}
__host__ __device__ inline size_t acts_bytes(int TT, int K) { return (size_t) TT * K + (size_t) TT * (K / 32) * 8; }

// rows ys[0..n) (rows 0..n-1 when ys is null) of q8_1 activations (36-byte blocks) into LDS: a thread per (row, block)
__device__ inline void stage_q8_1(const Acts& a, const uint8_t* __restrict__ xq, const int* ys, int n) {
    const int nb = a.K / 32;
    for (int it = threadIdx.x; it < n * nb; it += blockDim.x) {
        const int j = it / nb, b = it % nb;
        const uint8_t* blk = xq + ((size_t) (ys ? ys[j] : j) * nb + b) * Q81_BYTES;
        const int* src = reinterpret_cast<const int*>(blk + 4);
        int w[8], s = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            w[k] = src[k];
            s = dot4(w[k], 0x01010101, s);
        }
        int4* dst = reinterpret_cast<int4*>(a.q + (size_t) j * a.K + 32 * b);
        dst[0] = make_int4(w[0], w[1], w[2], w[3]);
        dst[1] = make_int4(w[4], w[5], w[6], w[7]);
        a.d[j * nb + b] = h2f(*reinterpret_cast<const uint16_t*>(blk));
        a.s[j * nb + b] = s;
    }
}

// h = silu(gate) * up of gu rows ys[0..n) (rows 0..n-1 when ys is null; [gate (K) | up (K)]) as q8_1 in LDS (k_moe_h,
// src/moe.cuh:284-295): a half-wave per (row, 32 columns)
__device__ inline void stage_swiglu(const Acts& a, const float* __restrict__ gu, const int* ys, int n) {
    const int nb = a.K / 32, hw = threadIdx.x / 32, l = threadIdx.x % 32, nhw = blockDim.x / 32;
    for (int it = hw; it < n * nb; it += nhw) {
        const int j = it / nb, b = it % nb;
        const float* g = gu + (size_t) (ys ? ys[j] : j) * 2 * a.K;
        const float xi = silu_f(g[32 * b + l]) * g[a.K + 32 * b + l];
        const float amax = group_max<32>(fabsf(xi));
        const float d = amax / 127.0f;
        const int q = amax == 0.0f ? 0 : (int) roundf(xi / d);
        const int s = group_isum<32>(q);
        a.q[(size_t) j * a.K + 32 * b + l] = (int8_t) q;
        if (l == 0) {
            a.d[j * nb + b] = h2f(f2h(d));
            a.s[j * nb + b] = s;
        }
    }
}

// ------------------------------------------------------------------------------------------------ Q4_K
// Q5_K (Q5): the same lanes and combine on 5-bit values, the fifth bits from the qh pieces of the lane's super-block
template <int GPL, bool Q5 = false> struct Q4kRow {
    uint4 q0[GPL], q1[GPL];
    uint4 h[GPL];
    uint4 qh0[Q5 ? GPL : 1], qh1[Q5 ? GPL : 1];
    float d[GPL], dmin[GPL], sc0[GPL], m0[GPL], sc1[GPL], m1[GPL];
    // the loads alone (issue several rows' before any prepare, so that their latencies overlap)
    // P: the planar store's planes (Q4kPlanes), or any view with the same accessors (one row staged in LDS)
    template <typename PL> __device__ __forceinline__ void issue(const PL& P, int row, int C, int l8) {
#pragma unroll
        for (int i = 0; i < GPL; ++i) {
            q0[i] = *reinterpret_cast<const uint4*>(P.nib16(row, C, 16 * i + l8));
            q1[i] = *reinterpret_cast<const uint4*>(P.nib16(row, C, 16 * i + 8 + l8));
            h[i] = *reinterpret_cast<const uint4*>(P.hdr16(row, C, 2 * i + (l8 >> 2)));
            if constexpr (Q5) {
                qh0[i] = *reinterpret_cast<const uint4*>(P.qh16(row, C, 2 * (2 * i + (l8 >> 2))));
                qh1[i] = *reinterpret_cast<const uint4*>(P.qh16(row, C, 2 * (2 * i + (l8 >> 2)) + 1));
            }
        }
    }
    // the block headers decoded: d, dmin and this lane's two sub-blocks' 6-bit scales and mins
    __device__ __forceinline__ void prepare(int l8) {
#pragma unroll
        for (int i = 0; i < GPL; ++i) {
            d[i] = h2f((uint16_t) (h[i].x & 0xffff));
            dmin[i] = h2f((uint16_t) (h[i].x >> 16));
            q4k_scale_min(h[i], 2 * (l8 & 3), sc0[i], m0[i]);
            q4k_scale_min(h[i], 2 * (l8 & 3) + 1, sc1[i], m1[i]);
        }
    }
    __device__ __forceinline__ void load(const Q4kPlanes& P, int row, int C, int l8) {
        issue(P, row, C, l8);
        prepare(l8);
    }
    // prepare() and dot(a, 0, l8) in one pass: a group's header decoded as the group is reached, so the work on the
    // first groups overlaps the arrival of the later ones (the same values as prepare() then dot())
    __device__ __forceinline__ float dot1(const Acts& a, int l8) {
        float tmp = 0.f;
#pragma unroll
        for (int i = 0; i < GPL; ++i) {
            d[i] = h2f((uint16_t) (h[i].x & 0xffff));
            dmin[i] = h2f((uint16_t) (h[i].x >> 16));
            q4k_scale_min(h[i], 2 * (l8 & 3), sc0[i], m0[i]);
            q4k_scale_min(h[i], 2 * (l8 & 3) + 1, sc1[i], m1[i]);
            tmp += group(a, 0, l8, i);
        }
        return tmp;
    }
    // group i of this lane's share of row . activation row j
    __device__ __forceinline__ float group(const Acts& a, int j, int l8, int i) const {
        const int kb0 = (2 * i + (l8 >> 2)) * 8 + 2 * (l8 & 3);
        const int4 a00 = a.q4(j, kb0)[0], a01 = a.q4(j, kb0)[1], a10 = a.q4(j, kb0 + 1)[0], a11 = a.q4(j, kb0 + 1)[1];
        const unsigned qw[8] = {q0[i].x, q0[i].y, q0[i].z, q0[i].w, q1[i].x, q1[i].y, q1[i].z, q1[i].w};
        const int al[8] = {a00.x, a00.y, a00.z, a00.w, a01.x, a01.y, a01.z, a01.w};
        const int ah[8] = {a10.x, a10.y, a10.z, a10.w, a11.x, a11.y, a11.z, a11.w};
        int dl = 0, dh = 0;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            unsigned lo = qw[w] & 0x0F0F0F0Fu, hi = (qw[w] >> 4) & 0x0F0F0F0Fu;
            if constexpr (Q5) {
                const unsigned hw = w < 4 ? (&qh0[i].x)[w] : (&qh1[i].x)[w - 4];
                const int jg = l8 & 3;
                lo |= ((hw >> (2 * jg)) & 0x01010101u) << 4;
                hi |= ((hw >> (2 * jg + 1)) & 0x01010101u) << 4;
            }
            dl = dot4((int) lo, al[w], dl);
            dh = dot4((int) hi, ah[w], dh);
        }
        const int nb = a.K / 32;
        const float d8l = a.d[j * nb + kb0], d8h = a.d[j * nb + kb0 + 1];
        const float sl = (float) a.s[j * nb + kb0], sh = (float) a.s[j * nb + kb0 + 1];
        return d[i] * (d8l * (sc0[i] * (float) dl) + d8h * (sc1[i] * (float) dh)) -
               dmin[i] * (d8l * (m0[i] * sl) + d8h * (m1[i] * sh));
    }
    // this lane's share of row . activation row j
    __device__ __forceinline__ float dot(const Acts& a, int j, int l8) const {
        float tmp = 0.f;
#pragma unroll
        for (int i = 0; i < GPL; ++i) tmp += group(a, j, l8, i);
        return tmp;
    }
};

// ------------------------------------------------------------------------------------------------ Q8_0
template <int BPL> struct Q80Row {
    uint4 qa[BPL], qb[BPL];
    uint32_t dh[BPL];   // (32-bit: a 16-bit register half would be filled by a load that waits for the other half's)
    float dw[BPL];
    template <typename PL> __device__ __forceinline__ void issue(const PL& P, int row, int C, int l16) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            qa[i] = *reinterpret_cast<const uint4*>(P.q16(row, C, 32 * i + l16));
            qb[i] = *reinterpret_cast<const uint4*>(P.q16(row, C, 32 * i + 16 + l16));
            dh[i] = *P.dof(row, C, l16 + 16 * i);
        }
    }
    __device__ __forceinline__ void prepare(int) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            // (opaque: the conversion stays here, where the caller put it, instead of rising to the load and making
            // every later request of the caller wait for this one)
            asm volatile("" : "+v"(dh[i]));
            dw[i] = h2f((uint16_t) dh[i]);
        }
    }
    __device__ __forceinline__ void load(const Q80Planes& P, int row, int C, int l16) {
        issue(P, row, C, l16);
        prepare(l16);
    }
    __device__ __forceinline__ float dot1(const Acts& a, int l16) {
        prepare(l16);
        return dot(a, 0, l16);
    }
    __device__ __forceinline__ float dot(const Acts& a, int j, int l16) const {
        float acc = 0.f;
        const int nb = a.K / 32;
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const int b = l16 + 16 * i;
            const int4 a0 = a.q4(j, b)[0], a1 = a.q4(j, b)[1];
            int s = dot4((int) qa[i].x, a0.x, 0);
            s = dot4((int) qa[i].y, a0.y, s);
            s = dot4((int) qa[i].z, a0.z, s);
            s = dot4((int) qa[i].w, a0.w, s);
            s = dot4((int) qb[i].x, a1.x, s);
            s = dot4((int) qb[i].y, a1.y, s);
            s = dot4((int) qb[i].z, a1.z, s);
            s = dot4((int) qb[i].w, a1.w, s);
            acc += (dw[i] * a.d[j * nb + b]) * (float) s;
        }
        return acc;
    }
};

// ------------------------------------------------------------------------------------------------ Q4_0, Q5_1
// bits 0..3 of t to bit 4 of bytes 0..3
__device__ __forceinline__ uint32_t spread4(uint32_t t) {
    return ((t & 1u) << 4) | ((t & 2u) << 11) | ((t & 4u) << 18) | ((t & 8u) << 25);
}
// The Q8_0 lanes (16 a row, lane l16 the blocks l16 + 16 i in order).  Per block the exact integer dot of the values
// (Q5_1: the fifth bit of value l is qh bit l) with the activation block, then Q4_0 (d_w d_a) (sum - 8 s), Q5_1
// (d_w d_a) sum + (m_w d_a) s, with s the block's integer activation sum.
template <int BPL, int TYPE> struct NbRow {
    uint4 q[BPL];
    uint32_t sv[BPL];   // Q4_0: f16 d (low half); Q5_1: f16 d | f16 m << 16
    uint32_t qh[TYPE == SFNX_Q5_1 ? BPL : 1];
    float dw[BPL], mw[BPL];
    template <typename PL> __device__ __forceinline__ void issue(const PL& P, int row, int C, int l16) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const int b = l16 + 16 * i;
            q[i] = *reinterpret_cast<const uint4*>(P.q16(row, C, b));
            if constexpr (TYPE == SFNX_Q4_0) {
                sv[i] = *reinterpret_cast<const uint16_t*>(P.d_of(row, C, b));
            } else {
                sv[i] = *reinterpret_cast<const uint32_t*>(P.dm_of(row, C, b));
                qh[i] = *reinterpret_cast<const uint32_t*>(P.qh_of(row, C, b));
            }
        }
    }
    __device__ __forceinline__ void prepare(int) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            dw[i] = h2f((uint16_t) (sv[i] & 0xffff));
            mw[i] = TYPE == SFNX_Q5_1 ? h2f((uint16_t) (sv[i] >> 16)) : 0.f;
        }
    }
    __device__ __forceinline__ void load(const NbPlanes& P, int row, int C, int l16) {
        issue(P, row, C, l16);
        prepare(l16);
    }
    __device__ __forceinline__ float dot1(const Acts& a, int l16) {
        prepare(l16);
        return dot(a, 0, l16);
    }
    __device__ __forceinline__ float dot(const Acts& a, int j, int l16) const {
        float acc = 0.f;
        const int nb = a.K / 32;
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const int b = l16 + 16 * i;
            const int4 a0 = a.q4(j, b)[0], a1 = a.q4(j, b)[1];
            const unsigned qw[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
            const int al[4] = {a0.x, a0.y, a0.z, a0.w}, ah[4] = {a1.x, a1.y, a1.z, a1.w};
            int sum = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                unsigned lo = qw[w] & 0x0F0F0F0Fu, hi = (qw[w] >> 4) & 0x0F0F0F0Fu;
                if constexpr (TYPE == SFNX_Q5_1) {
                    lo |= spread4(qh[i] >> (4 * w));
                    hi |= spread4(qh[i] >> (16 + 4 * w));
                }
                sum = dot4((int) lo, al[w], sum);
                sum = dot4((int) hi, ah[w], sum);
            }
            const float da = a.d[j * nb + b];
            const int sa = a.s[j * nb + b];
            if constexpr (TYPE == SFNX_Q4_0) acc += (dw[i] * da) * (float) (sum - 8 * sa);
            else acc += (dw[i] * da) * (float) sum + (mw[i] * da) * (float) sa;
        }
        return acc;
    }
};

// ------------------------------------------------------------------------------------------------ dense Q8_0 (q8s)
// The shared expert's dense Q8_0 rows as the reference computes them (src/dense.cuh:24-154 q8s_block): 32 lanes a
// row, lane L the 16-column halves c = 16 L + 512 i in order, acc_L = fmaf(d_w d_a, sum of the 16 products, acc_L),
// then v += shfl_xor(v, o) for o = 16 .. 1.  Here LPR physical lanes carry the 32 logical ones, L = ln + LPR k, and
// fold theirs in the butterfly's order (xor 16 and 8 are k ^ 2 and k ^ 1 for LPR 8, xor 16 is k ^ 1 for LPR 16), so
// group_sum<LPR> of the result finishes exactly the reference's sum.  Weights in the reference's split layout
// (Q8sPlanes): logical lane L's i-th 16 values are columns 512 i + 16 L of the row, block b = 16 i + L / 2, so the 32
// lanes of a row read 512 contiguous bytes.  Read straight from memory (the shared expert is one job of a launch; no
// register copy of the row is kept).
// The same sums from registers: issue() loads a row's values for the lane's logical lanes (NI = C / 512 each), dot()
// forms the lane's partial in q8s_dot's order.
template <int LPR, int NI> struct Q8sRow {
    static constexpr int NL = 32 / LPR;
    uint4 w[NL][NI];
    uint16_t dh[NL][NI];
    __device__ __forceinline__ void issue(const Q8sPlanes& P, int row, int C, int ln) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int k = 0; k < NL; ++k) {
                const int L = ln + LPR * k;
                w[k][i] = *reinterpret_cast<const uint4*>(P.q16(row, C, 512 * i + 16 * L));
                dh[k][i] = *P.dof(row, C, 16 * i + L / 2);
            }
    }
    __device__ __forceinline__ float dot(const Acts& a, int j, int ln) const {
        const int nb = a.K / 32;
        float acc[NL];
#pragma unroll
        for (int k = 0; k < NL; ++k) acc[k] = 0.f;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int k = 0; k < NL; ++k) {
                const int L = ln + LPR * k, h = L & 1, b = 16 * i + L / 2;
                const int4 av = a.q4(j, b)[h];
                int s = dot4((int) w[k][i].x, av.x, 0);
                s = dot4((int) w[k][i].y, av.y, s);
                s = dot4((int) w[k][i].z, av.z, s);
                s = dot4((int) w[k][i].w, av.w, s);
                acc[k] = fmaf(h2f(dh[k][i]) * a.d[j * nb + b], (float) s, acc[k]);
            }
        if constexpr (NL == 4) return (acc[0] + acc[2]) + (acc[1] + acc[3]);
        else if constexpr (NL == 2) return acc[0] + acc[1];
        else return acc[0];
    }
};

template <int LPR> __device__ __forceinline__ float q8s_dot(const Q8sPlanes& P, int row, int C, int ln, const Acts& a, int j) {
    static_assert(LPR == 8 || LPR == 16 || LPR == 32, "q8s lanes");
    constexpr int NL = 32 / LPR;
    const int nb = C / 32;
    float acc[NL];
#pragma unroll
    for (int k = 0; k < NL; ++k) acc[k] = 0.f;
    for (int i = 0; i < C / 512; ++i) {
#pragma unroll
        for (int k = 0; k < NL; ++k) {
            const int L = ln + LPR * k, h = L & 1, b = 16 * i + L / 2;
            const uint4 w = *reinterpret_cast<const uint4*>(P.q16(row, C, 512 * i + 16 * L));
            const float dw = h2f(*P.dof(row, C, b));
            const int4 av = a.q4(j, b)[h];
            int s = dot4((int) w.x, av.x, 0);
            s = dot4((int) w.y, av.y, s);
            s = dot4((int) w.z, av.z, s);
            s = dot4((int) w.w, av.w, s);
            acc[k] = fmaf(dw * a.d[j * nb + b], (float) s, acc[k]);
        }
    }
    if constexpr (NL == 4) return (acc[0] + acc[2]) + (acc[1] + acc[3]);
    else if constexpr (NL == 2) return acc[0] + acc[1];
    else return acc[0];
}

}  // namespace sfnx
