// The hyper-connection read that feeds the MoE half its input (src/hc.cuh:13-380 k_hc, src/kernels.cu:1054-1090
// hc_read): HC residual streams of N columns are folded with the last half's output, normalised, mixed through a
// low-rank pair of dense Q8_0 matrices (down [LR][HC N], up [HC N][LR]) and averaged into `mixed`, the MoE layer's
// input, with its q8_1 form for the expert dots.  Per row t:
//   R' = R + bo * 2 sigm(inj_prev / HC) per stream (when bo), xs = R' w_norm
//   K_A  (slice s of 512 columns, group of 32 rows): the slice's square sums of R' (32-value butterflies, then the 16
//        groups in order), xs as int8 per 32 (float d = amax / 127), each down row's partial dot (8 lanes, lane j the
//        8-value chunks 8 q + j in order, acc = fmaf(d_w d_x, dot8, acc), then xor 1, 2, 4) and the bf16 inject rows'
//        partial dots on xs itself
//   K_B  rs_c = 1 / sqrt(stream c's square sum / N + eps); lo_r = silu(sum_c fmaf(rs_c, sum_s part) / HC) as int8 per
//        32; inject_c the same combine without silu
//   K_C  (32 columns): up row c N + i: per 32-block b of lo, (d_w d_lo) dot32, folded as the reference's 16-lane xor
//        butterfly folds them (lane b holds block b; partners 1, 2, 4, 8);
//        mixed_i = sum_c sigm(up) ((R'_c,i w_norm) rs_c) / HC, R <- R', mixed as q8_1
// The reference runs the three parts in one launch with two grid barriers; here they are three launches, which cost
// less than a grid barrier on this part (a kernel boundary in a graph ~1.6 us, a 256-workgroup barrier ~2.8 us).
#include "common.hpp"

namespace sfnx {
namespace {

constexpr int HS = 512;              // columns of a slice
constexpr int HA_THREADS = 256;      // K_A: 32 rows x 8 lanes
constexpr int HA_ROWS = HA_THREADS / 8;
constexpr int HC_COLS = 32;          // K_C: 32 columns a block
constexpr int HC_THREADS = 512;
constexpr int HC_MAX = 8;            // streams
constexpr int LR_MAX = 512;          // 16 lanes x 32
constexpr int HCLR_MAX = 2048;       // HC LR: a K_C block's up rows (32 columns of every stream) in 64 KB of LDS

struct HcLayout {
    size_t part, ssp, loq, lod, rs, total;
};
// pieces laid out for windows of SFNX_MAXT rows whatever a call's T, so one workspace serves every window size
HcLayout hc_layout(int N, int HC, int LR) {
    constexpr size_t T = SFNX_MAXT;
    const size_t NS = (size_t) HC * N / HS, ROWS = (size_t) LR + HC;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t r = o;
        o += (bytes + 255) / 256 * 256;
        return r;
    };
    HcLayout L;
    L.part = take(T * NS * ROWS * 4);
    L.ssp = take(T * NS * 4);
    L.loq = take(T * LR);
    L.lod = take(T * (LR / 32) * 4);
    L.rs = take(T * HC * 4);
    L.total = o;
    return L;
}

struct HcArgs {
    float* R;
    const float* bo;
    const float* inj_prev;
    const float* w_norm;
    const int8_t* dq;
    const uint16_t* dd;
    const int8_t* uq;
    const uint16_t* ud;
    const uint16_t* w_inj;
    float eps;
    float* mixed;
    float* inject;
    uint8_t* xq;
    int T, N, HC, LR;
    float* part;   // [T][NS][LR + HC]
    float* ssp;    // [T][NS]
    int8_t* loq;   // [T][LR]
    float* lod;    // [T][LR / 32]
    float* rs;     // [T][HC]
};

// the xor butterfly in the reference's order for its hc sums: partner 1, then 2, 4, ... (v += shfl_xor(v, o))
template <int G> __device__ __forceinline__ float sum_up(float v) {
    if constexpr (G >= 2) v += lane_xor<1>(v);
    if constexpr (G >= 4) v += lane_xor<2>(v);
    if constexpr (G >= 8) v += lane_xor<4>(v);
    if constexpr (G >= 16) v += lane_xor<8>(v);
    return v;
}

// R' = R + bo 2 sigm(inj_prev / HC) per stream: hc_write's fold (src/kernels.cu:1493-1498) as src/hc.cuh:68-72
// applies it, fmaf(bo, 2 sigm(.), R), in K_A (its slice) and K_C (its columns), the same bits in both.

// one 32-value block to int8 with a float scale (src/hc.cuh:60-66), a half-wave per block
__device__ __forceinline__ void q8_block32(float v, int8_t* q, float* d) {
    const int l = threadIdx.x % 32;
    const float amax = group_max<32>(fabsf(v));
    const float sc = amax / 127.0f;
    q[l] = amax == 0.0f ? (int8_t) 0 : (int8_t) roundf(v / sc);
    if (l == 0) *d = sc;
}

// ------------------------------------------------------------------------------------------------ K_A
// windows of more than one row run 4 groups of HA_THREADS threads a block: group g takes its share of the rows in the
// slice's set-up and rows g, g + HA_TG, ... in the dots (each output's lanes and order as with one group)
template <int TT> constexpr int ha_tg() { return TT >= 4 ? 4 : 1; }
template <int TT>
__global__ void __launch_bounds__(HA_THREADS * ha_tg<TT>()) k_hc_down(HcArgs a) {
    constexpr int TG = ha_tg<TT>();
    __shared__ __align__(16) float xs[TT][HS];
    __shared__ __align__(16) int8_t xq[TT][HS];
    __shared__ float xd[TT][HS / 32];
    __shared__ float red[TT][HS / 32];
    const int T = a.T, s = blockIdx.x, grp = blockIdx.y, tid = threadIdx.x % HA_THREADS, tg = threadIdx.x / HA_THREADS;
    const int D = a.HC * a.N;
    const int NS = D / HS, ROWS = a.LR + a.HC, col0 = s * HS, c = col0 / a.N, i0 = col0 % a.N;
    // this block's weight row, loaded first: 8 lanes a row, lane j the chunks 8 q + j
    const int row = grp * HA_ROWS + tid / 8, j = tid % 8;
    const bool dn_row = row < a.LR, inj_row = row >= a.LR && row < ROWS && a.w_inj != nullptr;
    uint2 wd[8];
    uint4 wi[8];
    float sc[8];
    if (dn_row) {
        const uint2* w2 = reinterpret_cast<const uint2*>(a.dq + (size_t) row * D + col0);
        const uint16_t* ds = a.dd + ((size_t) row * D + col0) / 32;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            wd[q] = w2[q * 8 + j];
            sc[q] = h2f(ds[(q * 8 + j) / 4]);
        }
    } else if (inj_row) {
        const uint4* w4 = reinterpret_cast<const uint4*>(a.w_inj + (size_t) (row - a.LR) * D + col0);
#pragma unroll
        for (int q = 0; q < 8; ++q) wi[q] = w4[q * 8 + j];
    }
    const float wn0 = a.w_norm[col0 + tid], wn1 = a.w_norm[col0 + HA_THREADS + tid];
    // R' of the slice into xs, the rows' loads (and the fold's inject logits) issued RB at a time: batch m, element k
    // is row RB / 2 m + k / 2, column tid + 256 (k % 2), so a thread takes each row's gate once
    static_assert(HS == 2 * HA_THREADS, "two columns of a slice a thread");
    constexpr int RB = TG > 1 ? 2 * (TT / TG) : 8;   // a group's rows of a window in one batch
    for (int t0 = tg * (RB / 2); t0 < T; t0 += TG * (RB / 2)) {
        float r[RB], b[RB], g[RB / 2];
#pragma unroll
        for (int k = 0; k < RB; ++k) {
            const int t = t0 + k / 2, x = tid + HA_THREADS * (k % 2);
            if (t < T) {
                r[k] = a.R[(size_t) t * D + col0 + x];
                if (a.bo) {
                    b[k] = a.bo[(size_t) t * a.N + i0 + x];
                    if (k % 2 == 0) g[k / 2] = a.inj_prev[t * a.HC + c];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < RB / 2; ++k)
            if (a.bo && t0 + k < T) g[k] = 2.0f * sigm_f(g[k] / (float) a.HC);
#pragma unroll
        for (int k = 0; k < RB; ++k) {
            const int t = t0 + k / 2, x = tid + HA_THREADS * (k % 2);
            if (t < T) xs[t][x] = a.bo ? fmaf(b[k], g[k / 2], r[k]) : r[k];
        }
    }
    __syncthreads();
    // the square sums (row group 0 only): 32 consecutive columns a half-wave; then xs = R' w_norm
    const int hw = tid / 32;
#pragma unroll
    for (int t0 = 0; t0 < TT; t0 += TG) {
        const int t = t0 + tg;
        if (t >= T) break;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int x = h * HA_THREADS + tid;
            const float r = xs[t][x];
            if (grp == 0) {
                const float v = group_sum<32>(r * r);
                if (tid % 32 == 0) red[t][h * (HA_THREADS / 32) + hw] = v;
            }
            xs[t][x] = r * (h ? wn1 : wn0);
        }
    }
    __syncthreads();
    if (grp == 0 && tg == 0 && tid < T) {
        float v = 0.f;
        for (int w = 0; w < HS / 32; ++w) v += red[tid][w];
        a.ssp[(size_t) tid * NS + s] = v;
    }
    // xs as int8 per 32 (q8_block32's arithmetic: an exact maximum, then each value on its own): 8 threads a block,
    // 4 consecutive values each, so a pass covers 32 blocks
    for (int q = (int) threadIdx.x / 8; q < T * (HS / 32); q += TG * HA_THREADS / 8) {
        const int t = q / (HS / 32), b = q % (HS / 32), l8 = tid % 8;
        const float4 v = *reinterpret_cast<const float4*>(&xs[t][32 * b + 4 * l8]);
        const float amax = group_max<8>(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        const float sc = amax / 127.0f;
        const float vv[4] = {v.x, v.y, v.z, v.w};
        uint32_t pk = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) pk |= (uint32_t) (uint8_t) (amax == 0.0f ? (int8_t) 0 : (int8_t) roundf(vv[k] / sc)) << (8 * k);
        *reinterpret_cast<uint32_t*>(&xq[t][32 * b + 4 * l8]) = pk;
        if (l8 == 0) xd[t][b] = sc;
    }
    __syncthreads();
    if (row >= ROWS) return;   // whole 8-lane groups: the butterfly stays inside live groups
#pragma unroll
    for (int t0 = 0; t0 < TT; t0 += TG) {
        const int t = t0 + tg;
        if (t >= T) break;
        float acc = 0.f;
        if (dn_row) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int ch = q * 8 + j;
                const int2 xv = *reinterpret_cast<const int2*>(&xq[t][ch * 8]);
                const int d8 = dot4((int) wd[q].y, xv.y, dot4((int) wd[q].x, xv.x, 0));
                acc = fmaf(sc[q] * xd[t][ch / 4], (float) d8, acc);
            }
        } else if (inj_row) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int ch = q * 8 + j;
                const uint32_t h[4] = {wi[q].x, wi[q].y, wi[q].z, wi[q].w};
                const float* x = &xs[t][ch * 8];
                float e = __uint_as_float(h[0] << 16) * x[0];
                e = e + __uint_as_float(h[0] & 0xffff0000u) * x[1];
#pragma unroll
                for (int m = 1; m < 4; ++m) {
                    e = e + __uint_as_float(h[m] << 16) * x[2 * m];
                    e = e + __uint_as_float(h[m] & 0xffff0000u) * x[2 * m + 1];
                }
                acc = acc + e;
            }
        }
        acc = sum_up<8>(acc);
        if (j == 0) a.part[((size_t) t * NS + s) * ROWS + row] = acc;
    }
}

// ------------------------------------------------------------------------------------------------ K_B
// The combine of row r for token t (src/hc.cuh:251-289): rs_c = 1 / sqrt(stream c's slice square sums in order / N +
// eps), then sum_c fmaf(rs_c, stream c's slice partials in order, sum).  The square sums and the partials are loaded
// together, 32 slices at a time (one round trip for the reference's 20); rsv receives rs_c.
__device__ __forceinline__ float hc_combine(const HcArgs& a, int t, int r, float (&rsv)[HC_MAX]) {
    const int NS = a.HC * a.N / HS, SPS = a.N / HS, ROWS = a.LR + a.HC;
    float vs = 0.f, p = 0.f, sum = 0.f;
    int ss = 0, c = 0;   // slice within the stream, stream
    for (int q0 = 0; q0 < NS; q0 += 32) {
        float sv[32], pv[32];
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const int q = q0 + k;
            sv[k] = q < NS ? a.ssp[(size_t) t * NS + q] : 0.f;
            pv[k] = q < NS ? a.part[((size_t) t * NS + q) * ROWS + r] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            if (q0 + k >= NS) break;
            vs += sv[k];
            p += pv[k];
            if (++ss == SPS) {
                const float rc = 1.0f / sqrtf(vs / (float) a.N + a.eps);
#pragma unroll
                for (int cc = 0; cc < HC_MAX; ++cc)
                    if (cc == c) rsv[cc] = rc;
                sum = fmaf(rc, p, sum);
                vs = 0.f;
                p = 0.f;
                ss = 0;
                ++c;
            }
        }
    }
    return sum;
}

// item (t, b): b < LR / 32 a block of lo, b == LR / 32 the inject rows; a half-wave each
__global__ void __launch_bounds__(256) k_hc_reduce(HcArgs a) {
    const int NB = a.LR / 32, items = a.T * (NB + 1), l = threadIdx.x % 32;
    const int it = blockIdx.x * 8 + threadIdx.x / 32;
    if (it >= items) return;   // whole half-waves leave together
    const int t = it / (NB + 1), b = it % (NB + 1);
    const bool inj = b == NB;
    if (inj && (a.w_inj == nullptr || a.inject == nullptr)) return;
    float rsv[HC_MAX];
    const float sum = hc_combine(a, t, inj ? a.LR + min(l, a.HC - 1) : 32 * b + l, rsv);
    if (b == 0 && l < a.HC) {
#pragma unroll
        for (int c = 0; c < HC_MAX; ++c)
            if (c == l) a.rs[t * a.HC + l] = rsv[c];
    }
    if (inj) {
        if (l < a.HC) a.inject[t * a.HC + l] = sum;
    } else {
        q8_block32(silu_f(sum / (float) a.HC), a.loq + (size_t) t * a.LR + 32 * b, a.lod + (size_t) t * NB + b);
    }
}

// ------------------------------------------------------------------------------------------------ K_C
// 32 columns a block.  The block's up rows (HC streams x 32 columns, LR int8 each, and their scales) are staged in LDS;
// thread (c, column) then takes its row whole: the 32-blocks' (d_w d_lo) dot32 values, folded in the order of the
// reference's 16-lane xor butterfly (partner 1, 2, 4, 8; lanes past LR / 32 hold zeros), so no lane idles in a
// shuffle.  ONE (one row, LR + HC <= 512): the block makes lo and rs itself from the slices' partials (K_B's sums,
// the same bits), so the read takes two launches (src/hc.cuh's one-barrier form does the same).
// windows of 8 rows or more take 1024 threads a block (fewer dot items a thread)
template <int TT> constexpr int hc_up_threads() { return TT >= 8 ? 1024 : HC_THREADS; }
template <int TT, bool ONE>
__global__ void __launch_bounds__(hc_up_threads<TT>()) k_hc_up(HcArgs a) {
    constexpr int NTH = hc_up_threads<TT>();
    constexpr int PER = (TT * HC_MAX * HC_COLS + NTH - 1) / NTH;   // (t, c, column) items a thread
    __shared__ __align__(16) int8_t wq[HC_COLS * (HCLR_MAX + 16 * HC_MAX)];   // row rr = c 32 + column at rr (LR + 16)
    __shared__ float wsl[HC_COLS * HCLR_MAX / 32];
    __shared__ __align__(16) int8_t lq[TT][LR_MAX];
    __shared__ float ld[TT][LR_MAX / 32];
    __shared__ float rs[TT][HC_MAX];
    __shared__ float sg[TT][HC_MAX];
    __shared__ float gs[TT][HC_MAX][HC_COLS];
    __shared__ float ms[TT][HC_COLS];
    const int T = a.T, tid = threadIdx.x, NB = a.LR / 32, dc0 = blockIdx.x * HC_COLS;
    const int nitem = T * a.HC * HC_COLS, nrow = a.HC * HC_COLS;
    // every load of the block first: the up rows (16 bytes a thread at a time, 4 in flight), their scales, the
    // (t, c, column) items' R, bo and w_norm, then lo and rs
    {
        const int per_row = a.LR / 16, n16 = nrow * per_row;
#pragma unroll 4
        for (int e = tid; e < n16; e += NTH) {
            const int rr = e / per_row;
            const size_t u = (size_t) (rr / HC_COLS) * a.N + dc0 + rr % HC_COLS;
            reinterpret_cast<uint4*>(wq)[rr * (per_row + 1) + e % per_row] = reinterpret_cast<const uint4*>(a.uq + u * a.LR)[e % per_row];
        }
        for (int e = tid; e < nrow * NB; e += NTH) {
            const int rr = e / NB;
            wsl[e] = h2f(a.ud[((size_t) (rr / HC_COLS) * a.N + dc0 + rr % HC_COLS) * NB + e % NB]);
        }
    }
    float rv[PER], bv[PER], wn[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int e = tid + k * NTH;
        if (e < nitem) {
            const int cl = e % HC_COLS, c = (e / HC_COLS) % a.HC, t = e / (HC_COLS * a.HC), dc = dc0 + cl;
            rv[k] = a.R[(size_t) t * a.HC * a.N + (size_t) c * a.N + dc];
            if (a.bo) bv[k] = a.bo[(size_t) t * a.N + dc];
            wn[k] = a.w_norm[(size_t) c * a.N + dc];
        }
    }
    if constexpr (ONE) {
        const bool lo_row = tid < a.LR, inj_row = tid >= a.LR && tid < a.LR + a.HC && a.w_inj != nullptr;
        float rsv[HC_MAX];
        const float sum = lo_row || inj_row ? hc_combine(a, 0, tid, rsv) : 0.f;
        if (lo_row) q8_block32(silu_f(sum / (float) a.HC), &lq[0][32 * (tid / 32)], &ld[0][tid / 32]);
        if (inj_row && blockIdx.x == 0 && a.inject) a.inject[tid - a.LR] = sum;
        if (tid == 0) {
#pragma unroll
            for (int c = 0; c < HC_MAX; ++c)
                if (c < a.HC) {
                    rs[0][c] = rsv[c];
                    if (blockIdx.x == 0) a.rs[c] = rsv[c];
                }
        }
    } else {
        const int nq = T * a.LR / 4;
        for (int e0 = tid; e0 < nq; e0 += 4 * NTH) {
            int v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = e0 + k * NTH < nq ? reinterpret_cast<const int*>(a.loq)[e0 + k * NTH] : 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int e = e0 + k * NTH;
                if (e < nq) reinterpret_cast<int*>(&lq[e / (a.LR / 4)][0])[e % (a.LR / 4)] = v[k];
            }
        }
        if (tid < T * NB) ld[tid / NB][tid % NB] = a.lod[tid];
        if (tid < T * a.HC) rs[tid / a.HC][tid % a.HC] = a.rs[tid];
    }
    if (a.bo && tid < T * a.HC) sg[tid / a.HC][tid % a.HC] = 2.0f * sigm_f(a.inj_prev[tid] / (float) a.HC);
    __syncthreads();
    // item (t, c, column): the up row c 32 + column of the block against lo row t.  With few items (one row: 4 streams
    // x 32 columns for 512 threads) 4 consecutive lanes share an item, lane q taking leaves 4 q .. 4 q + 3 of the tree
    // below and lane exchanges (partners 1, then 2) making its last two levels: the same sums in the same pairs
    if (T * nrow * 4 <= NTH) {
        const int it = tid / 4, q = tid % 4;
        const bool live = it < T * nrow;
        const int t = live ? it / nrow : 0, rr = live ? it % nrow : 0, c = rr / HC_COLS, cl = rr % HC_COLS;
        auto blk = [&](int b) {
            if (b >= NB) return 0.f;
            const int4* wr = reinterpret_cast<const int4*>(wq + rr * (NB * 32 + 16) + 32 * b);
            const int4* xr = reinterpret_cast<const int4*>(&lq[t][32 * b]);
            const int4 w0 = wr[0], w1 = wr[1], x0 = xr[0], x1 = xr[1];
            int s = dot4(w0.x, x0.x, 0);
            s = dot4(w0.y, x0.y, s);
            s = dot4(w0.z, x0.z, s);
            s = dot4(w0.w, x0.w, s);
            s = dot4(w1.x, x1.x, s);
            s = dot4(w1.y, x1.y, s);
            s = dot4(w1.z, x1.z, s);
            s = dot4(w1.w, x1.w, s);
            return (wsl[rr * NB + b] * ld[t][b]) * (float) s;
        };
        float w = (blk(4 * q) + blk(4 * q + 1)) + (blk(4 * q + 2) + blk(4 * q + 3));
        w = w + lane_xor<1>(w);
        w = w + lane_xor<2>(w);
        if (live && q == 0) gs[t][c][cl] = w;
    } else
    for (int it = tid; it < T * nrow; it += NTH) {
        const int t = it / nrow, rr = it % nrow, c = rr / HC_COLS, cl = rr % HC_COLS;
        {
            // block b's (d_w d_lo) dot32, 0 past LR / 32 (the lanes of the reference's butterfly that hold no block)
            auto blk = [&](int b) {
                if (b >= NB) return 0.f;
                const int4* wr = reinterpret_cast<const int4*>(wq + rr * (NB * 32 + 16) + 32 * b);
                const int4* xr = reinterpret_cast<const int4*>(&lq[t][32 * b]);
                const int4 w0 = wr[0], w1 = wr[1], x0 = xr[0], x1 = xr[1];
                int s = dot4(w0.x, x0.x, 0);
                s = dot4(w0.y, x0.y, s);
                s = dot4(w0.z, x0.z, s);
                s = dot4(w0.w, x0.w, s);
                s = dot4(w1.x, x1.x, s);
                s = dot4(w1.y, x1.y, s);
                s = dot4(w1.z, x1.z, s);
                s = dot4(w1.w, x1.w, s);
                return (wsl[rr * NB + b] * ld[t][b]) * (float) s;
            };
            // the butterfly's tree: lane 0 ends with ((v0+v1)+(v2+v3)) + ... in pairs at distance 1, 2, 4, 8
            float u[8], w[4];
#pragma unroll
            for (int b = 0; b < 8; ++b) u[b] = blk(2 * b) + blk(2 * b + 1);
#pragma unroll
            for (int b = 0; b < 4; ++b) w[b] = u[2 * b] + u[2 * b + 1];
            gs[t][c][cl] = (w[0] + w[1]) + (w[2] + w[3]);
        }
    }
    __syncthreads();
    // item (t, c, column): the gate times the normalised stream, R <- R'
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int e = tid + k * NTH;
        if (e < nitem) {
            const int cl = e % HC_COLS, c = (e / HC_COLS) % a.HC, t = e / (HC_COLS * a.HC), dc = dc0 + cl;
            const float r = a.bo ? fmaf(bv[k], sg[t][c], rv[k]) : rv[k];
            if (a.bo) a.R[(size_t) t * a.HC * a.N + (size_t) c * a.N + dc] = r;
            gs[t][c][cl] = sigm_f(gs[t][c][cl]) * (r * wn[k] * rs[t][c]);
        }
    }
    __syncthreads();
    for (int e = tid; e < T * HC_COLS; e += NTH) {
        const int cl = e % HC_COLS, t = e / HC_COLS;
        float m = gs[t][0][cl];
        for (int c = 1; c < a.HC; ++c) m += gs[t][c][cl];
        m = m / (float) a.HC;
        a.mixed[(size_t) t * a.N + dc0 + cl] = m;
        ms[t][cl] = m;
    }
    if (a.xq == nullptr) return;
    __syncthreads();
    // mixed as q8_1 (k_quantize's arithmetic): a half-wave per row's block
    for (int t = tid / 32; t < T; t += NTH / 32) {
        const int l = tid % 32;
        const float xi = ms[t][l];
        const float amax = group_max<32>(fabsf(xi)), sum = group_sum<32>(xi);
        const float d = amax / 127.0f;
        uint8_t* blk = a.xq + ((size_t) t * (a.N / 32) + dc0 / 32) * Q81_BYTES;
        blk[4 + l] = (uint8_t) (int8_t) (amax == 0.0f ? 0 : (int) roundf(xi / d));
        if (l == 0) *reinterpret_cast<uint32_t*>(blk) = (uint32_t) f2h(d) | ((uint32_t) f2h(sum) << 16);
    }
}

template <int TT> void hc_launch(const HcArgs& a, hipStream_t s) {
    const int NS = a.HC * a.N / HS, RG = (a.LR + a.HC + HA_ROWS - 1) / HA_ROWS;
    k_hc_down<TT><<<dim3(NS, RG), HA_THREADS * ha_tg<TT>(), 0, s>>>(a);
    check(hipGetLastError(), "k_hc_down launch");
    if constexpr (TT == 1) {
        if (a.LR + a.HC <= HC_THREADS) {
            k_hc_up<TT, true><<<a.N / HC_COLS, hc_up_threads<TT>(), 0, s>>>(a);
            check(hipGetLastError(), "k_hc_up launch");
            return;
        }
    }
    {
        const int items = a.T * (a.LR / 32 + 1);
        k_hc_reduce<<<(items + 7) / 8, 256, 0, s>>>(a);
        check(hipGetLastError(), "k_hc_reduce launch");
        k_hc_up<TT, false><<<a.N / HC_COLS, hc_up_threads<TT>(), 0, s>>>(a);
    }
    check(hipGetLastError(), "k_hc_up launch");
}

}  // namespace
}  // namespace sfnx

using namespace sfnx;

extern "C" size_t sfnx_hc_workspace(int N, int HC, int LR, size_t* offsets) {
    const HcLayout L = hc_layout(N, HC, LR);
    if (offsets) {
        const size_t o[6] = {L.part, L.ssp, L.loq, L.lod, L.rs, L.total};
        for (int i = 0; i < 6; ++i) offsets[i] = o[i];
    }
    return L.total;
}

extern "C" int sfnx_hc_read(float* R, const float* bo, const float* inj_prev, const float* w_norm, const void* down_q,
                            const void* down_d, const void* up_q, const void* up_d, const void* w_inj, float eps,
                            float* mixed, float* inject, void* xq, int T, int N, int HC, int LR, void* ws,
                            size_t ws_bytes, void* st) {
    return guarded("sfnx_hc_read", [&] {
        require(R && w_norm && down_q && down_d && up_q && up_d && mixed && ws, "null argument");
        require(!bo || inj_prev, "bo needs inj_prev (the last half's inject logits)");
        require(T >= 1 && T <= SFNX_MAXT, "T out of range (1..16)");
        require(N > 0 && N % HS == 0, "N must be a positive multiple of 512");
        require(HC >= 1 && HC <= HC_MAX, "HC must be 1..8");
        require(LR > 0 && LR % 32 == 0 && LR <= LR_MAX, "LR must be a multiple of 32, at most 512");
        require(HC * LR <= HCLR_MAX, "HC LR must be at most 2048");
        const HcLayout L = hc_layout(N, HC, LR);
        require(ws_bytes >= L.total, "workspace smaller than sfnx_hc_workspace()");
        char* w = (char*) ws;
        HcArgs a{R, bo, inj_prev, w_norm, (const int8_t*) down_q, (const uint16_t*) down_d, (const int8_t*) up_q,
                 (const uint16_t*) up_d, (const uint16_t*) w_inj, eps, mixed, inject, (uint8_t*) xq, T, N, HC, LR,
                 (float*) (w + L.part), (float*) (w + L.ssp), (int8_t*) (w + L.loq), (float*) (w + L.lod),
                 (float*) (w + L.rs)};
        hipStream_t s = stream_of(st);
        if (T == 1) hc_launch<1>(a, s);
        else if (T <= 4) hc_launch<4>(a, s);
        else hc_launch<16>(a, s);
    });
}
