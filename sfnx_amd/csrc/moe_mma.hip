// The prompt path's routed experts on the matrix cores (src/moe_mma.cuh, src/moe_mma.cu:324-354): per BigJob (one
// expert, up to 64 token rows) and 512 of the expert's weight rows, out[job.out[m]][row] = sum_k w16[row][k] x16[m][k]
// with f16 weights (Q4_K: hfma2(q, f16(d sc), f16(-(dmin m))); Q8_0: hmul2(q, d)), f16 activations and fp32 accumulation,
// on v_mfma_f32_32x32x16_f16.
//
// Layout on gfx950 (wave64): a block is 16 wavefronts (4 a SIMD, 128 registers each); each wavefront owns 32 weight rows
// and dequantizes them straight from the planar store into the MFMA's B operand.  The K loop runs over 512-column runs
// of 8 steps, cut into chunks (Q4_K: 4 steps, one super-block; Q8_0: 2 steps): lane (n = l % 32, h = l / 32) holds row
// n's 16-byte pieces of the chunk's steps for lane-half h, and each step's 16 bytes are exactly the lane's 4 x 8 MFMA
// k-slots (the columns are permuted; the sum does not depend on the order of k).  The store's 32-row tiling makes every
// such request whole 128-byte lines.  The job's activation rows for the run sit in LDS and feed the A operand with the
// same permutation.  Weight chunks stream through two register slots; the next run's activations come into the other
// LDS buffer by asynchronous global -> LDS copies.  D[token][row] leaves as 128-byte runs of consecutive rows.
#include "mv.hpp"

namespace sfnx {
namespace {


typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));

// SiLU on the prompt path as the reference compiles it (src/moe_mma.cuh:382-388 under --use_fast_math: __expf is
// 2^(x log2 e) on the hardware exp2, the division a reciprocal): x rcp(1 + 2^(-x log2 e))
__device__ __forceinline__ float silu_fast(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.44269504088896340736f));
}

constexpr int MM_WAVES = 16, MM_THREADS = MM_WAVES * WAVE, MM_BM = 32 * MM_WAVES;   // 512 weight rows a block
__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

// bytes 0, 1 (SEL 0) or 2, 3 (SEL 1) of w as two f16 values 1024 + byte (0x64 above each byte)
template <int SEL> __device__ __forceinline__ half2v bytes_1024(uint32_t w) {
    return as_h2(__builtin_amdgcn_perm(0x64646464u, w, SEL == 0 ? 0x05010400u : 0x05030402u));
}

// Q4_K: 16 bytes of a group's quants (b0..b15, low nibbles of sub-block 2jg, high of 2jg + 1) -> the 4 B fragments;
// Q5_K (qh given): the fifth bit of each value from bit j0 (low nibbles) or j0 + 1 (high) of the matching qh byte
__device__ __forceinline__ void deq_q4k(const uint4& q, half2v d1l, half2v nml, half2v d1h, half2v nmh, half8 (&b)[4],
                                        const uint4* qh = nullptr, int j0 = 0) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const uint32_t x[4] = {qh ? qh->x : 0u, qh ? qh->y : 0u, qh ? qh->z : 0u, qh ? qh->w : 0u};
    const half2v k1024 = {(_Float16) 1024.0f, (_Float16) 1024.0f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        // chunk c: low nibbles of bytes 8 c' .. 8 c' + 7 (c' = c % 2) for c < 2, high nibbles for c >= 2
        const int wi = 2 * (c % 2);
        const bool hi = c >= 2;
        const half2v d1 = hi ? d1h : d1l, nm = hi ? nmh : nml;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            uint32_t v = hi ? (w[wi + p] >> 4) & 0x0F0F0F0Fu : w[wi + p] & 0x0F0F0F0Fu;
            if (qh) v |= ((x[wi + p] >> (hi ? j0 + 1 : j0)) & 0x01010101u) << 4;
            const half2v q01 = bytes_1024<0>(v) - k1024, q23 = bytes_1024<1>(v) - k1024;
            const half2v r01 = __builtin_elementwise_fma(q01, d1, nm), r23 = __builtin_elementwise_fma(q23, d1, nm);
            b[c][4 * p + 0] = r01[0];
            b[c][4 * p + 1] = r01[1];
            b[c][4 * p + 2] = r23[0];
            b[c][4 * p + 3] = r23[1];
        }
    }
}

// Q8_0: a block's 32 signed quants (two 16-byte halves) -> 4 B fragments, hmul2(q, d)
__device__ __forceinline__ void deq_q80(const uint4& qa, const uint4& qb, half2v d, half8 (&b)[4]) {
    const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const half2v k1152 = {(_Float16) 1152.0f, (_Float16) 1152.0f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t v = w[2 * c + p] ^ 0x80808080u;   // q + 128 as bytes
            const half2v q01 = bytes_1024<0>(v) - k1152, q23 = bytes_1024<1>(v) - k1152;
            const half2v r01 = q01 * d, r23 = q23 * d;
            b[c][4 * p + 0] = r01[0];
            b[c][4 * p + 1] = r01[1];
            b[c][4 * p + 2] = r23[0];
            b[c][4 * p + 3] = r23[1];
        }
}

// One lane's raw weights for a chunk of a 512-column run (Q4_K: 4 steps of 64 columns, one super-block; Q8_0: 2 steps).
// Q4_K: 4 of the 16-byte halves h of the run's 8 groups (64 bytes of the lane's 128-byte half-line) and the chunk's
// super-block header; Q8_0: blocks 8 h + 2 c, 8 h + 2 c + 1 of the run's 16 (both 16-byte halves of each) and their two
// scales.  Step j of a run pairs lane-half 0's group / block j with lane-half 1's.
template <int TYPE> struct Chunk;
template <> struct Chunk<SFNX_Q4_K> {
    static constexpr int STEPS = 4, LOADS = 5;   // steps a chunk; load instructions a chunk
    uint4 q[4], hdr;
};
template <> struct Chunk<SFNX_Q5_K> {
    static constexpr int STEPS = 4, LOADS = 6;
    uint4 q[4], hdr, qh;   // qh: the super-block's qh bytes 16 h .. 16 h + 15 (the fifth bits of the lane's values)
};
template <> struct Chunk<SFNX_Q4_0> {
    static constexpr int STEPS = 4, LOADS = 5;
    uint4 q[4];   // blocks 8 h + 4 c .. + 3 of the run
    uint2 d;      // their four f16 d
};
template <> struct Chunk<SFNX_Q5_1> {
    static constexpr int STEPS = 4, LOADS = 6;
    uint4 q[4], dm, qh;   // the blocks' (f16 d, f16 m) and qh words
};
template <> struct Chunk<SFNX_Q8_0> {
    static constexpr int STEPS = 2, LOADS = 5;
    uint4 qa[2], qb[2];
    uint32_t d;
};

// Where chunk c (of the run's 8 / STEPS) of run r of the lane's row lies.
struct ChunkAt {
    const uint8_t* q;     // the first 16-byte piece (K-quants: nibbles; Q8_0: first halves); the next one a tile's pieces on
    const uint8_t* tail;  // K-quants: the super-block header; Q8_0: the two f16 scales
    const uint8_t* qh;    // Q5_K: the lane-half's qh piece
};
__device__ __forceinline__ ChunkAt chunk_at(const Chunk<SFNX_Q4_K>*, const uint8_t* mat, int R, int C, int row, int r, int c, int h) {
    const Q4kPlanes P = q4k_planes(mat, R, C);
    return ChunkAt{P.nib16(row, C, 16 * r + 8 * h + 4 * c), P.hdr16(row, C, 2 * r + c), nullptr};
}
__device__ __forceinline__ ChunkAt chunk_at(const Chunk<SFNX_Q5_K>*, const uint8_t* mat, int R, int C, int row, int r, int c, int h) {
    const KqPlanes P = q5k_planes(mat, R, C);
    return ChunkAt{P.nib16(row, C, 16 * r + 8 * h + 4 * c), P.hdr16(row, C, 2 * r + c), P.qh16(row, C, 2 * (2 * r + c) + h)};
}
// Q4_0 / Q5_1: step s of chunk c of run r, lane-half h is block 16 r + 8 h + 4 c + s of the row
template <int TYPE> __device__ __forceinline__ ChunkAt chunk_at_nb(const uint8_t* mat, int R, int C, int row, int r, int c, int h) {
    const NbPlanes P = nb_planes<TYPE>(mat, R, C);
    const int kb = 16 * r + 8 * h + 4 * c;
    if constexpr (TYPE == SFNX_Q4_0) return ChunkAt{P.q16(row, C, kb), P.d_of(row, C, kb), nullptr};
    else return ChunkAt{P.q16(row, C, kb), P.dm_of(row, C, kb), P.qh_of(row, C, kb)};
}
__device__ __forceinline__ ChunkAt chunk_at(const Chunk<SFNX_Q4_0>*, const uint8_t* mat, int R, int C, int row, int r, int c, int h) {
    return chunk_at_nb<SFNX_Q4_0>(mat, R, C, row, r, c, h);
}
__device__ __forceinline__ ChunkAt chunk_at(const Chunk<SFNX_Q5_1>*, const uint8_t* mat, int R, int C, int row, int r, int c, int h) {
    return chunk_at_nb<SFNX_Q5_1>(mat, R, C, row, r, c, h);
}
__device__ __forceinline__ ChunkAt chunk_at(const Chunk<SFNX_Q8_0>*, const uint8_t* mat, int R, int C, int row, int r, int c, int h) {
    const Q80Planes P = q80_planes(mat, R, C);
    return ChunkAt{P.q16(row, C, 32 * r + 8 * h + 2 * c), P.d16(row, C, 2 * r + h) + 4 * c, nullptr};
}
__device__ __forceinline__ void load_piece(Chunk<SFNX_Q4_K>& w, const ChunkAt& a, int s) {
    w.q[s] = *reinterpret_cast<const uint4*>(a.q + PIECE_STRIDE * s);
}
__device__ __forceinline__ void load_piece(Chunk<SFNX_Q5_K>& w, const ChunkAt& a, int s) {
    w.q[s] = *reinterpret_cast<const uint4*>(a.q + PIECE_STRIDE * s);
}
__device__ __forceinline__ void load_piece(Chunk<SFNX_Q4_0>& w, const ChunkAt& a, int s) {
    w.q[s] = *reinterpret_cast<const uint4*>(a.q + Q80_RT * 16 * s);
}
__device__ __forceinline__ void load_piece(Chunk<SFNX_Q5_1>& w, const ChunkAt& a, int s) {
    w.q[s] = *reinterpret_cast<const uint4*>(a.q + Q80_RT * 16 * s);
}
__device__ __forceinline__ void load_piece(Chunk<SFNX_Q8_0>& w, const ChunkAt& a, int s) {
    w.qa[s] = *reinterpret_cast<const uint4*>(a.q + Q80_RT * 16 * s);
    w.qb[s] = *reinterpret_cast<const uint4*>(a.q + Q80_RT * 16 * (16 + s));   // the blocks' second halves
}
__device__ __forceinline__ void load_tail(Chunk<SFNX_Q4_K>& w, const ChunkAt& a) { w.hdr = *reinterpret_cast<const uint4*>(a.tail); }
__device__ __forceinline__ void load_tail(Chunk<SFNX_Q5_K>& w, const ChunkAt& a) {
    w.hdr = *reinterpret_cast<const uint4*>(a.tail);
    w.qh = *reinterpret_cast<const uint4*>(a.qh);
}
__device__ __forceinline__ void load_tail(Chunk<SFNX_Q4_0>& w, const ChunkAt& a) { w.d = *reinterpret_cast<const uint2*>(a.tail); }
__device__ __forceinline__ void load_tail(Chunk<SFNX_Q5_1>& w, const ChunkAt& a) {
    w.dm = *reinterpret_cast<const uint4*>(a.tail);
    w.qh = *reinterpret_cast<const uint4*>(a.qh);
}
__device__ __forceinline__ void load_tail(Chunk<SFNX_Q8_0>& w, const ChunkAt& a) { w.d = *reinterpret_cast<const uint32_t*>(a.tail); }
template <int TYPE> constexpr bool tail_early();
// a chunk's requests in the order mma_chunk's refill makes them, so the compiler's count of requests in flight is the
// same for each slot on entry to the walk as on every later chunk, and its waits can count exactly
template <int TYPE> __device__ __forceinline__ void load_chunk(Chunk<TYPE>& w, const ChunkAt& a) {
    if constexpr (tail_early<TYPE>()) load_tail(w, a);
#pragma unroll
    for (int s = 0; s < Chunk<TYPE>::STEPS; ++s) load_piece(w, a, s);
    if constexpr (!tail_early<TYPE>()) load_tail(w, a);
}

// The 8 sub-blocks' f16(d sc) and f16(-(dmin m)) of a K-quant super-block header, all at once: the 6-bit values of
// q4k_scale_min as bytes (4 to a dword), 1024 + v as f16 through v_perm, minus 1024, times f16 d (or -dmin) in packed
// f16.  An f16 times a 6-bit integer is exact in fp32, so this single f16 rounding equals the f16 of the fp32 d * sc.
struct KScales {
    half2v D[4], N[4];   // D[k] = {f16(d sc_2k), f16(d sc_2k+1)}; N[k] the same of -(dmin m)
};
__device__ __forceinline__ KScales k_scales(const uint4& hd) {
    const uint32_t sc_lo = hd.y & 0x3F3F3F3Fu, m_lo = hd.z & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
    const uint32_t m_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t) (hd.x & 0xffff));
    const _Float16 nmin = -__builtin_bit_cast(_Float16, (uint16_t) (hd.x >> 16));
    const half2v dd = {d, d}, nn = {nmin, nmin}, k1024 = {(_Float16) 1024.0f, (_Float16) 1024.0f};
    KScales k;
    k.D[0] = (bytes_1024<0>(sc_lo) - k1024) * dd;
    k.D[1] = (bytes_1024<1>(sc_lo) - k1024) * dd;
    k.D[2] = (bytes_1024<0>(sc_hi) - k1024) * dd;
    k.D[3] = (bytes_1024<1>(sc_hi) - k1024) * dd;
    k.N[0] = (bytes_1024<0>(m_lo) - k1024) * nn;
    k.N[1] = (bytes_1024<1>(m_lo) - k1024) * nn;
    k.N[2] = (bytes_1024<0>(m_hi) - k1024) * nn;
    k.N[3] = (bytes_1024<1>(m_hi) - k1024) * nn;
    return k;
}
struct NoScales {};
template <int TYPE> __device__ __forceinline__ auto chunk_scales(const Chunk<TYPE>& w) {
    if constexpr (is_kquant(TYPE)) return k_scales(w.hdr);
    else return NoScales{};
}

// step s of a chunk as the 4 B fragments of its MFMAs
__device__ __forceinline__ void dequant_step(const Chunk<SFNX_Q4_K>& w, int s, half8 (&b)[4], const KScales& k) {
    const half2v D = k.D[s], N = k.N[s];
    deq_q4k(w.q[s], half2v{D[0], D[0]}, half2v{N[0], N[0]}, half2v{D[1], D[1]}, half2v{N[1], N[1]}, b);
}
__device__ __forceinline__ void dequant_step(const Chunk<SFNX_Q5_K>& w, int s, half8 (&b)[4], const KScales& k) {
    const half2v D = k.D[s], N = k.N[s];
    deq_q4k(w.q[s], half2v{D[0], D[0]}, half2v{N[0], N[0]}, half2v{D[1], D[1]}, half2v{N[1], N[1]}, b, &w.qh, 2 * s);
}
// Q4_0 / Q5_1: a block's 16 quant bytes (value l in the low nibble of byte l, l + 16 in the high) -> the 4 B
// fragments, fragment c holding values 8 c .. 8 c + 7; Q4_0 hmul2(q - 8, d), Q5_1 hfma2(q, d, m) with the fifth bits
template <int TYPE>
__device__ __forceinline__ void deq_nb(const uint4& q, uint32_t dm, uint32_t qh, half8 (&b)[4]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const half2v d = {__builtin_bit_cast(_Float16, (uint16_t) (dm & 0xffff)), __builtin_bit_cast(_Float16, (uint16_t) (dm & 0xffff))};
    const half2v m = {__builtin_bit_cast(_Float16, (uint16_t) (dm >> 16)), __builtin_bit_cast(_Float16, (uint16_t) (dm >> 16))};
    const half2v off = TYPE == SFNX_Q4_0 ? half2v{(_Float16) 1032.0f, (_Float16) 1032.0f} : half2v{(_Float16) 1024.0f, (_Float16) 1024.0f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const bool hi = c >= 2;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int wi = 2 * (c % 2) + p;   // the dword: values 4 wi .. 4 wi + 3 (+ 16 for the high nibbles)
            uint32_t v = hi ? (w[wi] >> 4) & 0x0F0F0F0Fu : w[wi] & 0x0F0F0F0Fu;
            if constexpr (TYPE == SFNX_Q5_1) v |= spread4(qh >> ((hi ? 16 : 0) + 4 * wi));
            const half2v q01 = bytes_1024<0>(v) - off, q23 = bytes_1024<1>(v) - off;
            half2v r01, r23;
            if constexpr (TYPE == SFNX_Q4_0) {
                r01 = q01 * d;
                r23 = q23 * d;
            } else {
                r01 = __builtin_elementwise_fma(q01, d, m);
                r23 = __builtin_elementwise_fma(q23, d, m);
            }
            b[c][4 * p + 0] = r01[0];
            b[c][4 * p + 1] = r01[1];
            b[c][4 * p + 2] = r23[0];
            b[c][4 * p + 3] = r23[1];
        }
    }
}
__device__ __forceinline__ void dequant_step(const Chunk<SFNX_Q4_0>& w, int s, half8 (&b)[4], NoScales) {
    deq_nb<SFNX_Q4_0>(w.q[s], (s < 2 ? w.d.x : w.d.y) >> (16 * (s % 2)), 0u, b);
}
__device__ __forceinline__ void dequant_step(const Chunk<SFNX_Q5_1>& w, int s, half8 (&b)[4], NoScales) {
    deq_nb<SFNX_Q5_1>(w.q[s], (&w.dm.x)[s], (&w.qh.x)[s], b);
}
__device__ __forceinline__ void dequant_step(const Chunk<SFNX_Q8_0>& w, int s, half8 (&b)[4], NoScales) {
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t) (w.d >> (16 * s)));
    deq_q80(w.qa[s], w.qb[s], half2v{d, d}, b);
}

// column (within the run's 512) where MFMA k-chunk c of step j starts for lane-half h
template <int TYPE> __device__ __forceinline__ int run_col(int j, int c, int h) {
    if constexpr (is_kquant(TYPE)) return 64 * j + (c < 2 ? 16 * h + 8 * c : 32 + 16 * h + 8 * (c - 2));
    else return 256 * h + 32 * j + 8 * c;
}

#ifndef MM_SLOTS
#define MM_SLOTS 2   // weight chunks a wavefront keeps in registers: the one being dotted and the ones in flight
#endif
constexpr int MM_RUN = 512, MM_XLD = MM_RUN + 8;   // columns a run; LDS row pitch (16 bytes past the run: rows shift banks)
constexpr size_t MM_XBUF = 64 * MM_XLD;              // halves in one activation buffer

// run r of the job's activation rows into an LDS buffer by asynchronous global -> LDS copies (no registers): wavefront w
// of W moves rows w * 64 / W .. (w + 1) * 64 / W - 1, a row of 512 halves a copy (64 lanes x 16 bytes); rows past n are
// left as they are (they only feed output rows that are never stored)
template <int W>
__device__ __forceinline__ void load_x_async(_Float16* buf, const _Float16* __restrict__ x, int ldx, const int* ys, int n,
                                             int r, int wave, int lane) {
    constexpr int XR = 64 / W;
#pragma unroll
    for (int i = 0; i < XR; ++i) {
        const int m = wave * XR + i;
        if (m < n) lds_copy_async<16>(x + (size_t) ys[m] * ldx + MM_RUN * r + 8 * lane, buf + (size_t) m * MM_XLD);
    }
}

// One chunk's steps on one wavefront's 32 weight rows: per step the 4 B fragments are dequantized from the registers
// (VALU), then each of the 4 k-pieces takes the activation fragment from LDS and one MFMA per 32-token tile.  Several
// wavefronts share each SIMD, so one's dequantization overlaps another's matrix work.
//
// The registers of the chunk refill with the chunk `next` (k + MM_SLOTS; the last chunks request the final one again,
// so every chunk issues the same requests) as they free up: piece s right after step s is dequantized, the Q4_K
// header once its scales are decoded (the other types use their tail in every step, so it follows the last step).
// Each request then has almost two chunks' time before it is needed, not one, from the same registers.
template <int TYPE> constexpr bool tail_early() { return TYPE == SFNX_Q4_K; }
template <int TYPE, int NT>
__device__ __forceinline__ void mma_chunk(Chunk<TYPE>& w, int cj, const _Float16* xb, int nn, int h, float16v (&acc)[NT],
                                          const ChunkAt& next) {
    constexpr int S = Chunk<TYPE>::STEPS;
    const auto sc = chunk_scales(w);
    if constexpr (tail_early<TYPE>()) load_tail(w, next);
#pragma unroll
    for (int s = 0; s < S; ++s) {
        half8 b[4];
        dequant_step(w, s, b, sc);
        load_piece(w, next, s);
        const int j = cj * S + s;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            half8 a[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) a[t] = *reinterpret_cast<const half8*>(xb + (size_t) (32 * t + nn) * MM_XLD + run_col<TYPE>(j, c, h));
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[t], b[c], acc[t], 0, 0, 0);
        }
    }
    if constexpr (!tail_early<TYPE>()) load_tail(w, next);
}

// The chunk walk shared by both kernels.  A wavefront's work is `tiles` row tiles of 32 rows (row_of(it)), each over
// the nr runs of 512 columns, each run CPR chunks: chunk k = (tile, run, chunk-in-run) in that order.  Weights stream
// through two register slots, chunk k + 2 requested piece by piece while chunk k is dotted.  The job's activation rows for a run
// sit in one of two LDS buffers; run r + 1's are requested (global -> LDS, no registers) when run r starts, so each
// run start waits only for them, not for the weight chunks requested after them (CPR chunks of LOADS requests each).
// tile_done(it, acc) takes a tile's accumulators (and they are cleared for the next tile); the last tile's stay in acc.
template <int TYPE, int NT, int W, typename RowOf, typename TileDone>
__device__ __forceinline__ void chunk_walk(const uint8_t* mat, int R, int C, int tiles, RowOf row_of, int wave, int lane,
                                           const int* ys, int n, const _Float16* __restrict__ x, _Float16* xs,
                                           float16v (&acc)[NT], TileDone tile_done) {
    constexpr int CPR = 8 / Chunk<TYPE>::STEPS, LD = Chunk<TYPE>::LOADS;
    static_assert(CPR % MM_SLOTS == 0, "a run's chunks fill the register slots evenly, so every slot steps every time");
    const int h = lane / 32, nn = lane % 32, nr = C / MM_RUN, per_tile = nr * CPR, NK = tiles * per_tile;
    auto at = [&](int k) {
        const int it = k / per_tile, rc = k % per_tile;
        return chunk_at((const Chunk<TYPE>*) nullptr, mat, R, C, row_of(it), rc / CPR, rc % CPR, h);
    };
    load_x_async<W>(xs, x, C, ys, n, 0, wave, lane);
    Chunk<TYPE> w[MM_SLOTS];
#pragma unroll
    for (int i = 0; i < MM_SLOTS; ++i)
        if (i < NK) load_chunk(w[i], at(i));
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = float16v{};
    // one chunk: the run's activations first when the chunk starts a run, then the dots, then the tile's end
    auto step = [&](Chunk<TYPE>& w, int k) {
        const int rc = k % per_tile, r = rc / CPR, cj = rc % CPR, rg = k / CPR;   // rg: runs walked so far
        _Float16* xb = xs + (size_t) (nr > 1 ? rg & 1 : 0) * MM_XBUF;
        if (cj == 0 && (nr > 1 || k == 0)) {
            // this run's rows: requested before the weight requests of the CPR chunks since (the copies are not
            // tracked by the compiler, so this wait is theirs).  Then the block barrier without the memory fence of
            // __syncthreads, which would drain the weight chunks in flight: every wavefront's rows landed, and every
            // wavefront's reads of the previous run's buffer fed its matrix instructions
            if (k == 0) vm_wait<0>();
            else vm_wait<CPR * LD>();
            lds_barrier();
            if (nr > 1 && k + per_tile / nr < NK) load_x_async<W>(xs + (size_t) ((rg + 1) & 1) * MM_XBUF, x, C, ys, n, (r + 1) % nr, wave, lane);
        }
        mma_chunk<TYPE, NT>(w, cj, xb, nn, h, acc, at(min(k + MM_SLOTS, NK - 1)));
        if (rc == per_tile - 1 && k + 1 < NK) {
            tile_done(k / per_tile, acc);
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = float16v{};
        }
    };
    for (int k0 = 0; k0 < NK; k0 += MM_SLOTS) {
#pragma unroll
        for (int i = 0; i < MM_SLOTS; ++i) step(w[i], k0 + i);   // refills w[i] with chunk k + MM_SLOTS
    }
}

// D[token][row] of a tile: lane (nn, h), value q at token 8 (q / 4) + 4 h + q % 4 of 32-token tile t
__device__ __forceinline__ int acc_token(int t, int q, int h) { return 32 * t + 8 * (q / 4) + 4 * h + q % 4; }

// rows: ys[0..n) (activation rows) and outs[0..n) (output rows, ldo floats apart), n <= 32 NT; the block's rows are G
// tiles of 32 W
template <int TYPE, int NT, int W>
__device__ __forceinline__ void mma_job(const uint8_t* mat, int R, int C, int row0, int G, int wave, int lane,
                                        const int* ys, const int* outs, int n, const _Float16* __restrict__ x,
                                        _Float16* xs, float* __restrict__ out, int ldo) {
    const int h = lane / 32, nn = lane % 32;
    auto row_of = [&](int it) { return row0 + it * 32 * W + wave * 32 + nn; };
    auto store = [&](int it, const float16v (&acc)[NT]) {
        const int row = row_of(it);
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int m = acc_token(t, q, h);
                if (m < n) out[(size_t) outs[m] * ldo + row] = acc[t][q];
            }
    };
    float16v acc[NT];
    chunk_walk<TYPE, NT, W>(mat, R, C, G, row_of, wave, lane, ys, n, x, xs, acc, store);
    store(G - 1, acc);
}

// The gate|up projection: a block owns FF indices f0 .. f0 + 255; wavefronts 0-7 take the gate rows f0 + 32 w + .,
// wavefronts 8-15 the matching up rows ff + f0 + 32 (w - 8) + .  Epilogue: gu (fp32 rows, when given) and h16 =
// f16(silu(gate) up) (when given), from the same accumulators, so the fused form equals moe_gate_up_mma followed by
// swiglu_h16 bit for bit.  The up accumulators reach the gate wavefronts through LDS.
constexpr int MM_FF = MM_BM / 2;   // FF indices a gate|up block owns
template <int TYPE, int NT>
__device__ __forceinline__ void mma_gu_job(const uint8_t* mat, int ff, int C, int f0, int wave, int lane,
                                           const sfnx_bigjob& jb, const _Float16* __restrict__ x, _Float16* xs,
                                           float* __restrict__ gu, _Float16* __restrict__ h16) {
    const int h = lane / 32, nn = lane % 32, R = 2 * ff, up = wave >= MM_WAVES / 2, fl = 32 * (wave % (MM_WAVES / 2)) + nn;
    const int row = (up ? ff : 0) + f0 + fl;
    float16v res[NT];
    chunk_walk<TYPE, NT, MM_WAVES>(mat, R, C, 1, [&](int) { return row; }, wave, lane, jb.y, jb.n, x, xs, res,
                         [](int, const float16v (&)[NT]) {});
    if (gu) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int m = acc_token(t, q, h);
                if (m < jb.n) gu[(size_t) jb.out[m] * R + row] = res[t][q];
            }
    }
    if (h16) {
        // up rows as fp32 [token][256] at the start of LDS, then h as f16 [token][256 (+8)] after them, then 16-byte
        // stores of whole 512-byte row pieces
        constexpr int HLD = MM_FF + 8;
        float* us = reinterpret_cast<float*>(xs);
        _Float16* hs = xs + 2 * 64 * MM_FF;
        __syncthreads();   // every wavefront is past the last run's activations
        if (up)
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int q = 0; q < 16; ++q) us[acc_token(t, q, h) * MM_FF + fl] = res[t][q];
        __syncthreads();
        if (!up)
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int m = acc_token(t, q, h);
                    hs[m * HLD + fl] = (_Float16) (silu_fast(res[t][q]) * us[m * MM_FF + fl]);
                }
        __syncthreads();
        for (int i = threadIdx.x; i < jb.n * (MM_FF / 8); i += MM_THREADS) {
            const int m = i / (MM_FF / 8), c = i % (MM_FF / 8);
            *reinterpret_cast<uint4*>(h16 + (size_t) jb.out[m] * ff + f0 + 8 * c) = *reinterpret_cast<const uint4*>(hs + m * HLD + 8 * c);
        }
    }
}

// Workgroup b runs on XCD b % 8.  The grid is 1-D: a job's row slices and MM_XG consecutive jobs (an expert's jobs
// are consecutive) go to one XCD and are dispatched together, so an expert's weight rows come from HBM once for all its
// jobs in the group and from that XCD's L2 for the rest, and the slices share the staged activation rows.
constexpr int MM_XG = 4;
__device__ __forceinline__ void xcd_job(int b, int nsl, int& slice, int& job) {
    const int x = b % XCDS, k = b / XCDS, m = k / nsl;
    slice = k % nsl;
    job = MM_XG * (XCDS * (m / MM_XG) + x) + m % MM_XG;
}
inline int xcd_grid(int nsl, int njobs_cap) { return nsl * ((njobs_cap + XCDS * MM_XG - 1) / (XCDS * MM_XG)) * XCDS * MM_XG; }

template <int TYPE>
__global__ void __launch_bounds__(MM_THREADS) k_moe_mma_gu(const uint8_t* __restrict__ A, size_t sa, int ff, int C,
                                                          const sfnx_bigjob* __restrict__ jobs, const int* __restrict__ njobs,
                                                          const _Float16* __restrict__ x, float* __restrict__ gu,
                                                          _Float16* __restrict__ h16) {
    int sl, ji;
    xcd_job(blockIdx.x, ff / MM_FF, sl, ji);
    if (ji >= *njobs) return;
    __shared__ sfnx_bigjob jb;
    extern __shared__ __align__(16) unsigned char xs_raw[];
    load_job(jb, jobs + ji);
    __syncthreads();
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const uint8_t* mat = expert_at(A, sa, jb.w);
    _Float16* xs = reinterpret_cast<_Float16*>(xs_raw);
    if (jb.n > 32) mma_gu_job<TYPE, 2>(mat, ff, C, sl * MM_FF, wave, lane, jb, x, xs, gu, h16);
    else mma_gu_job<TYPE, 1>(mat, ff, C, sl * MM_FF, wave, lane, jb, x, xs, gu, h16);
}

// The other projections (down, and gate|up shapes the paired kernel does not take): blocks of DN_WAVES wavefronts,
// two a compute unit when one run covers the input (one activation buffer), so one block's start (its activations
// and first weights in flight) overlaps the other's work.
// A dense matrix's prompt rows as the BigJobs of one "expert": job j takes rows 64 j .. 64 j + 63 of C to the same rows
__device__ __forceinline__ void dense_job(sfnx_bigjob& jb, int j, int C) {
    const int n = min(SFNX_PF_JOB, C - SFNX_PF_JOB * j);
    for (int m = threadIdx.x; m < SFNX_PF_JOB; m += blockDim.x) {
        const int t = m < n ? SFNX_PF_JOB * j + m : 0;
        jb.y[m] = t;
        jb.out[m] = t;
    }
    if (threadIdx.x == 0) {
        jb.w = 0;
        jb.n = n;
    }
}

constexpr int DN_WAVES = 8, DN_THREADS = DN_WAVES * WAVE, DN_BM = 32 * DN_WAVES;
template <int TYPE>
__global__ void __launch_bounds__(DN_THREADS, 4) k_moe_mma(const uint8_t* __restrict__ A, size_t sa, int R, int C, int G,
                                                       const sfnx_bigjob* __restrict__ jobs, const int* __restrict__ njobs,
                                                       const _Float16* __restrict__ x, float* __restrict__ out, int ldo,
                                                       int dense_c) {
    int sl, ji;
    xcd_job(blockIdx.x, R / (G * DN_BM), sl, ji);
    if (ji >= (dense_c > 0 ? (dense_c + SFNX_PF_JOB - 1) / SFNX_PF_JOB : *njobs)) return;
    __shared__ sfnx_bigjob jb;
    extern __shared__ __align__(16) unsigned char xs_raw[];
    if (dense_c > 0) dense_job(jb, ji, dense_c);
    else load_job(jb, jobs + ji);
    __syncthreads();
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const uint8_t* mat = expert_at(A, sa, jb.w);
    _Float16* xs = reinterpret_cast<_Float16*>(xs_raw);
    const int row0 = sl * G * DN_BM;
    if (jb.n > 32) mma_job<TYPE, 2, DN_WAVES>(mat, R, C, row0, G, wave, lane, jb.y, jb.out, jb.n, x, xs, out, ldo);
    else mma_job<TYPE, 1, DN_WAVES>(mat, R, C, row0, G, wave, lane, jb.y, jb.out, jb.n, x, xs, out, ldo);
}

// k_swiglu_h16 (src/moe_mma.cuh:382-388): h16 = f16(silu(gate) * up) of P rows [gate (ff) | up (ff)]
__global__ void k_swiglu_h16(const float* __restrict__ gu, int ff, int P, _Float16* __restrict__ h16) {
    const size_t n = (size_t) P * ff;
    for (size_t e = blockIdx.x * (size_t) blockDim.x + threadIdx.x; e < n; e += (size_t) gridDim.x * blockDim.x) {
        const size_t p = e / ff, i = e % ff;
        h16[e] = (_Float16) (silu_fast(gu[p * 2 * ff + i]) * gu[p * 2 * ff + ff + i]);
    }
}

__global__ void k_to_f16(const float* __restrict__ x, _Float16* __restrict__ y, size_t n) {
    for (size_t e = blockIdx.x * (size_t) blockDim.x + threadIdx.x; e < n; e += (size_t) gridDim.x * blockDim.x)
        y[e] = (_Float16) x[e];
}

constexpr size_t MM_LDS = 2 * MM_XBUF * sizeof(_Float16);


// out rows ldo floats apart (0: n_out); G: 256-row tiles a block walks (0: half of them, for routed jobs, which are many);
// dense_c > 0: no job list, the rows of one matrix (A) as jobs of 64 rows (dense_job)
void moe_mma(uint32_t type, const void* A, size_t sa, int n_in, int n_out, const sfnx_bigjob* jobs, const int* njobs,
             int njobs_cap, const void* x16, float* out, void* st, int ldo = 0, int G = 0, int dense_c = 0) {
    require(expert_type_ok(type), TYPE_MSG);
    require(n_in > 0 && n_in % 512 == 0, "expert input width must be a multiple of 512");
    require(n_out > 0 && n_out % DN_BM == 0, "expert rows must be a multiple of 256");
    require((n_out / DN_BM) % std::max(1, (n_out / DN_BM) / 2) == 0, "row groups must split evenly");
    require(stride_ok(sa, row_bytes(type, n_in) * (size_t) n_out), "expert stride smaller than a matrix");
    require(njobs_cap >= 0 && njobs_cap <= (1 << 20), "njobs_cap out of range");
    if (njobs_cap == 0) return;
    // tiles of 256 rows: two blocks a job (half the tiles each), for more blocks than compute units
    const int groups = n_out / DN_BM;
    if (G <= 0) G = std::max(1, groups / 2);
    require(groups % G == 0, "row groups must split evenly");
    if (ldo <= 0) ldo = n_out;
    const dim3 grid(xcd_grid(groups / G, njobs_cap));
    const size_t lds = (n_in == MM_RUN ? 1 : 2) * MM_XBUF * sizeof(_Float16);
    hipStream_t s = stream_of(st);
    if (type == SFNX_Q4_K)
        k_moe_mma<SFNX_Q4_K><<<grid, DN_THREADS, lds, s>>>((const uint8_t*) A, sa, n_out, n_in, G, jobs, njobs, (const _Float16*) x16, out, ldo, dense_c);
    else if (type == SFNX_Q5_K)
        k_moe_mma<SFNX_Q5_K><<<grid, DN_THREADS, lds, s>>>((const uint8_t*) A, sa, n_out, n_in, G, jobs, njobs, (const _Float16*) x16, out, ldo, dense_c);
    else if (type == SFNX_Q4_0)
        k_moe_mma<SFNX_Q4_0><<<grid, DN_THREADS, lds, s>>>((const uint8_t*) A, sa, n_out, n_in, G, jobs, njobs, (const _Float16*) x16, out, ldo, dense_c);
    else if (type == SFNX_Q5_1)
        k_moe_mma<SFNX_Q5_1><<<grid, DN_THREADS, lds, s>>>((const uint8_t*) A, sa, n_out, n_in, G, jobs, njobs, (const _Float16*) x16, out, ldo, dense_c);
    else
        k_moe_mma<SFNX_Q8_0><<<grid, DN_THREADS, lds, s>>>((const uint8_t*) A, sa, n_out, n_in, G, jobs, njobs, (const _Float16*) x16, out, ldo, dense_c);
}

void moe_mma_gu(uint32_t type, const void* A, size_t sa, int n_in, int ff, const sfnx_bigjob* jobs, const int* njobs,
                int njobs_cap, const void* x16, float* gu, uint16_t* h16, void* st) {
    require(expert_type_ok(type), TYPE_MSG);
    require(n_in > 0 && n_in % 512 == 0, "expert input width must be a multiple of 512");
    require(ff > 0 && ff % MM_FF == 0, "FF must be a multiple of 256");
    require(stride_ok(sa, row_bytes(type, n_in) * (size_t) (2 * ff)), "expert stride smaller than a matrix");
    require(njobs_cap >= 0 && njobs_cap <= (1 << 20), "njobs_cap out of range");
    if (njobs_cap == 0) return;
    const dim3 grid(xcd_grid(ff / MM_FF, njobs_cap));
    hipStream_t s = stream_of(st);
    if (type == SFNX_Q4_K)
        k_moe_mma_gu<SFNX_Q4_K><<<grid, MM_THREADS, MM_LDS, s>>>((const uint8_t*) A, sa, ff, n_in, jobs, njobs,
                                                                  (const _Float16*) x16, gu, (_Float16*) h16);
    else if (type == SFNX_Q5_K)
        k_moe_mma_gu<SFNX_Q5_K><<<grid, MM_THREADS, MM_LDS, s>>>((const uint8_t*) A, sa, ff, n_in, jobs, njobs,
                                                                  (const _Float16*) x16, gu, (_Float16*) h16);
    else if (type == SFNX_Q4_0)
        k_moe_mma_gu<SFNX_Q4_0><<<grid, MM_THREADS, MM_LDS, s>>>((const uint8_t*) A, sa, ff, n_in, jobs, njobs,
                                                                  (const _Float16*) x16, gu, (_Float16*) h16);
    else if (type == SFNX_Q5_1)
        k_moe_mma_gu<SFNX_Q5_1><<<grid, MM_THREADS, MM_LDS, s>>>((const uint8_t*) A, sa, ff, n_in, jobs, njobs,
                                                                  (const _Float16*) x16, gu, (_Float16*) h16);
    else
        k_moe_mma_gu<SFNX_Q8_0><<<grid, MM_THREADS, MM_LDS, s>>>((const uint8_t*) A, sa, ff, n_in, jobs, njobs,
                                                                  (const _Float16*) x16, gu, (_Float16*) h16);
}

}  // namespace
}  // namespace sfnx

using namespace sfnx;


extern "C" int sfnx_moe_gate_up_mma(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_bigjob* jobs,
                                    const int* njobs, int njobs_cap, const uint16_t* xh, float* gu, void* st) {
    return guarded("sfnx_moe_gate_up_mma", [&] {
        if (n_out % (2 * MM_FF) == 0 && n_in > MM_RUN)
            moe_mma_gu(type, A, sa, n_in, n_out / 2, jobs, njobs, njobs_cap, xh, gu, nullptr, st);
        else
            moe_mma(type, A, sa, n_in, n_out, jobs, njobs, njobs_cap, xh, gu, st);
    });
}

extern "C" int sfnx_moe_gate_up_swiglu_mma(const void* A, size_t sa, uint32_t type, int n_in, int ff, const sfnx_bigjob* jobs,
                                           const int* njobs, int njobs_cap, const uint16_t* xh, uint16_t* h16, void* st) {
    return guarded("sfnx_moe_gate_up_swiglu_mma", [&] {
        require(h16 != nullptr, "h16 is required");
        moe_mma_gu(type, A, sa, n_in, ff, jobs, njobs, njobs_cap, xh, nullptr, h16, st);
    });
}

extern "C" int sfnx_moe_down_mma(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_bigjob* jobs,
                                 const int* njobs, int njobs_cap, const uint16_t* h16, float* part, void* st) {
    return guarded("sfnx_moe_down_mma", [&] { moe_mma(type, A, sa, n_in, n_out, jobs, njobs, njobs_cap, h16, part, st); });
}

extern "C" int sfnx_swiglu_h16(const float* gu, int ffs, int P, uint16_t* h16, void* st) {
    return guarded("sfnx_swiglu_h16", [&] {
        require(ffs > 0, "FF must be positive");
        if (P <= 0) return;
        const size_t n = (size_t) P * ffs;
        k_swiglu_h16<<<(unsigned) std::min<size_t>((n + 255) / 256, 16384), 256, 0, stream_of(st)>>>(gu, ffs, P, (_Float16*) h16);
    });
}

extern "C" int sfnx_to_f16(const float* x, uint16_t* y, size_t n, void* st) {
    return guarded("sfnx_to_f16", [&] {
        if (!n) return;
        k_to_f16<<<(unsigned) std::min<size_t>((n + 255) / 256, 16384), 256, 0, stream_of(st)>>>(x, (_Float16*) y, n);
    });
}

extern "C" int sfnx_pf_dense(const sfnx_q8s* W, int rows, int cols, const uint16_t* xh, int C, float* out, int ldo,
                             void* wk, size_t wk_bytes, void* st) {
    return guarded("sfnx_pf_dense", [&] {
        require(W != nullptr && W->q != nullptr && W->d != nullptr && xh != nullptr && out != nullptr && wk != nullptr,
                "null pointer");
        require(rows > 0 && rows % DN_BM == 0 && cols > 0 && cols % MM_RUN == 0, "rows must be a multiple of 256, cols of 512");
        require(C >= 1 && C <= (1 << 20) && ldo >= rows, "C out of range, or ldo smaller than rows");
        require(wk_bytes >= q8s_planar_bytes(rows, cols), "wk smaller than the matrix's Q8_0 staging (rows * cols * 34 / 32 bytes)");
        // the reference converts the matrix into its staging buffer (k_q8s_f16 into p.wh) and multiplies in one f16
        // GEMM with fp32 results (pf_dense_xh, cublasGemmEx); here the staging is the planar Q8_0 layout, run as one
        // expert of the matrix-core kernels, whose weights are the same f16 values (hmul2(q, d)), dotted in fp32 on
        // v_mfma_f32_32x32x16_f16, its rows the jobs of 64 rows each block makes for itself
        hipStream_t s = stream_of(st);
        q8s_to_planar(*W, rows, cols, wk, s);
        const int nj = (C + SFNX_PF_JOB - 1) / SFNX_PF_JOB;
        const size_t sa = q8s_planar_bytes(rows, cols);
        // one 256-row tile a block: few jobs, so every tile is a block of its own
        moe_mma(SFNX_Q8_0, wk, sa, cols, rows, nullptr, nullptr, nj, xh, out, st, ldo, 1, C);
    });
}
