// The prompt path's routed experts on the matrix cores (src/moe_mma.cuh, src/moe_mma.cu:324-354): per BigJob (one
// expert, up to 64 token rows) and 256 of the expert's weight rows, out[job.out[m]][row] = sum_k w16[row][k] x16[m][k]
// with f16 weights (Q4_K: hfma2(q, f16(d sc), f16(-(dmin m))); Q8_0: hmul2(q, d)), f16 activations and fp32 accumulation,
// on v_mfma_f32_32x32x16_f16.
//
// Layout on gfx950 (wave64): each wavefront owns 32 weight rows and dequantizes them straight from the planar store into
// the MFMA's B operand.  The K loop runs over 512-column runs of 8 steps: per run, lane (n = l % 32, h = l / 32) loads
// one whole 128-byte line of row n (Q4_K: the 16-byte halves h of the run's 8 groups; Q8_0: blocks 8 h .. 8 h + 7) and
// the step's columns are permuted so that each step's 16 bytes are exactly the lane's 4 x 8 MFMA k-slots (the sum does
// not depend on the order of k).  The job's activation rows for the run sit in LDS and feed the A operand with the same
// permutation; the next run's weights and activations are in flight (registers) while this run's 8 steps compute.
// D[token][row] leaves as 128-byte runs of consecutive rows.
#include "mv.hpp"

namespace sfnx {
namespace {

#ifdef SFNX_PHASE_PROF
__device__ unsigned long long g_mma_prof[512][20];   // wall-clock stamps of blocks (job < 512, slice 0)
#define MPROF(i) if (threadIdx.x == 0 && pj >= 0) g_mma_prof[pj][i] = wall_clock64();
#else
#define MPROF(i)
#endif

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int MM_WAVES = 8, MM_THREADS = MM_WAVES * WAVE, MM_BM = 32 * MM_WAVES;   // 256 weight rows a block
__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

// bytes 0, 1 (SEL 0) or 2, 3 (SEL 1) of w as two f16 values 1024 + byte (0x64 above each byte)
template <int SEL> __device__ __forceinline__ half2v bytes_1024(uint32_t w) {
    return as_h2(__builtin_amdgcn_perm(0x64646464u, w, SEL == 0 ? 0x05010400u : 0x05030402u));
}

// Q4_K: 16 bytes of a group's quants (b0..b15, low nibbles of sub-block 2jg, high of 2jg + 1) -> the 4 B fragments
__device__ __forceinline__ void deq_q4k(const uint4& q, half2v d1l, half2v nml, half2v d1h, half2v nmh, half8 (&b)[4]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const half2v k1024 = {(_Float16) 1024.0f, (_Float16) 1024.0f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        // chunk c: low nibbles of bytes 8 c' .. 8 c' + 7 (c' = c % 2) for c < 2, high nibbles for c >= 2
        const int wi = 2 * (c % 2);
        const bool hi = c >= 2;
        const half2v d1 = hi ? d1h : d1l, nm = hi ? nmh : nml;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t v = hi ? (w[wi + p] >> 4) & 0x0F0F0F0Fu : w[wi + p] & 0x0F0F0F0Fu;
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

// One lane's raw weights for a run of 512 columns (8 steps of 64): Q4_K: its 128-byte half-line of the row's run (the
// 16-byte halves h of the run's 8 groups) and the run's two super-block headers; Q8_0: blocks 8 h .. 8 h + 7 of the
// run's 16 (both 16-byte halves of each, contiguous) and their scales.  Step j pairs lane-half 0's group / block j with
// lane-half 1's.
template <int TYPE> struct RunW;
template <> struct RunW<SFNX_Q4_K> {
    uint4 q[8], hdr[2];
};
template <> struct RunW<SFNX_Q8_0> {
    uint4 qa[8], qb[8], d;
};

__device__ __forceinline__ void load_run(RunW<SFNX_Q4_K>& w, const uint8_t* mat, int R, int C, int row, int r, int h) {
    const Q4kPlanes P = q4k_planes(mat, R, C);
    const uint4* q = reinterpret_cast<const uint4*>(P.nib_row(row, C) + 512 / 2 * r + 128 * h);
#pragma unroll
    for (int j = 0; j < 8; ++j) w.q[j] = q[j];
    const uint4* hd = reinterpret_cast<const uint4*>(P.hdr_row(row, C) + 32 * r);
    w.hdr[0] = hd[0];
    w.hdr[1] = hd[1];
}
__device__ __forceinline__ void load_run(RunW<SFNX_Q8_0>& w, const uint8_t* mat, int R, int C, int row, int r, int h) {
    const Q80Planes P = q80_planes(mat, R, C);
    const uint4* qa = reinterpret_cast<const uint4*>(P.q + (size_t) row * C + 512 * r + 128 * h);
    const uint4* qb = reinterpret_cast<const uint4*>(P.q + (size_t) row * C + 512 * r + 256 + 128 * h);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        w.qa[j] = qa[j];
        w.qb[j] = qb[j];
    }
    w.d = *reinterpret_cast<const uint4*>(P.d + (size_t) row * (C / 32) + 16 * r + 8 * h);
}

__device__ __forceinline__ void dequant_step(const RunW<SFNX_Q4_K>& w, int j, half8 (&b)[4]) {
    const uint4 hd = w.hdr[j / 4];
    const float d = h2f((uint16_t) (hd.x & 0xffff)), dmin = h2f((uint16_t) (hd.x >> 16));
    const int jg = j % 4;
    float sc, m;
    q4k_scale_min(hd, 2 * jg, sc, m);
    const _Float16 d1l = (_Float16) (d * sc), nml = (_Float16) (-(dmin * m));
    q4k_scale_min(hd, 2 * jg + 1, sc, m);
    const _Float16 d1h = (_Float16) (d * sc), nmh = (_Float16) (-(dmin * m));
    deq_q4k(w.q[j], half2v{d1l, d1l}, half2v{nml, nml}, half2v{d1h, d1h}, half2v{nmh, nmh}, b);
}
__device__ __forceinline__ void dequant_step(const RunW<SFNX_Q8_0>& w, int j, half8 (&b)[4]) {
    const uint32_t dw[4] = {w.d.x, w.d.y, w.d.z, w.d.w};
    const uint16_t db = (uint16_t) (dw[j / 2] >> (16 * (j % 2)));
    const _Float16 d = __builtin_bit_cast(_Float16, db);
    deq_q80(w.qa[j], w.qb[j], half2v{d, d}, b);
}

// column (within the run's 512) where MFMA k-chunk c of step j starts for lane-half h
template <int TYPE> __device__ __forceinline__ int run_col(int j, int c, int h) {
    if constexpr (TYPE == SFNX_Q4_K) return 64 * j + (c < 2 ? 16 * h + 8 * c : 32 + 16 * h + 8 * (c - 2));
    else return 256 * h + 32 * j + 8 * c;
}

constexpr int MM_RUN = 512, MM_XLD = MM_RUN + 8;   // columns a run; LDS row pitch (16 bytes past the run: rows shift banks)
constexpr int MM_XROWS = 64 / MM_WAVES;             // activation rows a wavefront moves per run
constexpr size_t MM_XBUF = 64 * MM_XLD;              // halves in one activation buffer

// run r of the job's activation rows into an LDS buffer by asynchronous global -> LDS copies (no registers): wavefront w
// moves rows w * 8 .. w * 8 + 7, a row of 512 halves a copy (64 lanes x 16 bytes); rows past n are left as they are
// (they only feed output rows that are never stored)
template <int XR = MM_XROWS>
__device__ __forceinline__ void load_x_async(_Float16* buf, const _Float16* __restrict__ x, int ldx, const int* ys, int n,
                                             int r, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < XR; ++i) {
        const int m = wave * XR + i;
        if (m < n)
            __builtin_amdgcn_global_load_lds(x + (size_t) ys[m] * ldx + MM_RUN * r + 8 * lane,
                                             (__attribute__((address_space(3))) void*) (buf + (size_t) m * MM_XLD), 16, 0, 0);
    }
}
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }   // vmcnt(0), others unwaited

// One run's 8 steps of 64 columns on one wavefront's 32 weight rows: step j's activation fragments are read from LDS
// first, then step j + 1's weight fragments are dequantized (VALU, covering the LDS latency) interleaved with step j's
// MFMAs; the scheduling groups keep that order (1 MFMA, then a share of the VALU).
template <int TYPE, int NT>
__device__ __forceinline__ void mma_run(const RunW<TYPE>& w, const _Float16* xb, int nn, int h, float16v (&acc)[NT]) {
    half8 bc[4], bn[4];
    dequant_step(w, 0, bc);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        half8 ac[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                ac[t][c] = *reinterpret_cast<const half8*>(xb + (size_t) (32 * t + nn) * MM_XLD + run_col<TYPE>(j, c, h));
        if (j < 7) dequant_step(w, j + 1, bn);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ac[t][c], bc[c], acc[t], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 4 * NT, 0);   // the DS reads
        __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);       // VALU while they land
#pragma unroll
        for (int q = 0; q < 4 * NT; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // an MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 48 / (4 * NT), 0);
        }
        if (j < 7)
#pragma unroll
            for (int c = 0; c < 4; ++c) bc[c] = bn[c];
    }
}

// The block's rows are G groups of 256 (a wavefront's 32 rows each); per group the runs of 512 columns, per run 8
// steps of 64.  Weights stream one run ahead of the steps (registers); each run's activations come into the other LDS
// buffer while this one is read.  A single run (the down projection) is staged once for every group.
// rows: ys[0..n) (activation rows) and outs[0..n) (output rows), n <= 32 NT
template <int TYPE, int NT>
__device__ __forceinline__ void mma_job(const uint8_t* mat, int R, int C, int row0, int G, int wave, int lane,
                                        const int* ys, const int* outs, int n, const _Float16* __restrict__ x, int ldx,
                                        _Float16* xs, float* __restrict__ out, int pj) {
    (void) pj;   // the job's row of phase stamps in the instrumented build, or -1
    constexpr int XR = NT <= 2 ? MM_XROWS : 4 * NT;   // activation rows a wavefront stages
    const int h = lane / 32, nn = lane % 32, nr = C / MM_RUN, total = G * nr;
    auto row_of = [&](int it) { return row0 + (it / nr) * MM_BM + wave * 32 + nn; };
    RunW<TYPE> w, wn;
    load_x_async<XR>(xs, x, ldx, ys, n, 0, wave, lane);
    load_run(w, mat, R, C, row_of(0), 0, h);
    float16v acc[NT];
    for (int it = 0; it < total; ++it) {
        if (it < 16) { MPROF(2 + it) }
        const int r = it % nr;
        if (r == 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = float16v{};
        }
        // buffers alternate by iteration (one run staged for good when there is only one)
        _Float16* xb = xs + (size_t) (nr > 1 ? it & 1 : 0) * MM_XBUF;
        if (nr > 1 || it == 0) {
            wait_vmem();          // this run's activations (and the weights of this step, needed now anyway)
            __syncthreads();      // every wavefront's rows landed; every wavefront is past the previous run
            if (nr > 1 && it + 1 < total)
                load_x_async<XR>(xs + (size_t) ((it + 1) & 1) * MM_XBUF, x, ldx, ys, n, (r + 1) % nr, wave, lane);
        }
        if (it + 1 < total) load_run(wn, mat, R, C, row_of(it + 1), (it + 1) % nr, h);
        mma_run<TYPE, NT>(w, xb, nn, h, acc);
        if (r == nr - 1) {
            // D[token][row]: lane (nn, h), value q at token 8 (q / 4) + 4 h + q % 4 of the tile
            const int row = row_of(it);
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int m = 32 * t + 8 * (q / 4) + 4 * h + q % 4;
                    if (m < n) out[(size_t) outs[m] * R + row] = acc[t][q];
                }
        }
        w = wn;
    }
}

// The gate|up projection by pairs of row groups: a block owns FF indices f0 .. f0 + 255, i.e. gate rows f0 + . and the
// matching up rows ff + f0 + .; the runs of 512 columns are the outer loop and each run's activations are staged once
// for both groups.  Epilogue: gu (fp32 rows, when given) and h16 = f16(silu(gate) up) (when given), from the same
// accumulators, so the fused form equals moe_gate_up_mma followed by swiglu_h16 bit for bit.
template <int TYPE, int NT>
__device__ __forceinline__ void mma_gu_job(const uint8_t* mat, int ff, int C, int f0, int wave, int lane,
                                           const sfnx_bigjob& jb, const _Float16* __restrict__ x, _Float16* xs,
                                           float* __restrict__ gu, _Float16* __restrict__ h16) {
    const int h = lane / 32, nn = lane % 32, nr = C / MM_RUN, R = 2 * ff, f = f0 + wave * 32 + nn;
    const int rows[2] = {f, ff + f};
    RunW<TYPE> w, wn;
    load_x_async(xs, x, C, jb.y, jb.n, 0, wave, lane);
    load_run(w, mat, R, C, rows[0], 0, h);
    float16v acc[2][NT];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[g][t] = float16v{};
    for (int r = 0; r < nr; ++r) {
        _Float16* xb = xs + (size_t) (r & 1) * MM_XBUF;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            if (g == 0) {
                wait_vmem();          // this run's activations and gate weights
                __syncthreads();      // every wavefront's rows landed; every wavefront is past the previous run
                if (r + 1 < nr) load_x_async(xs + (size_t) ((r + 1) & 1) * MM_XBUF, x, C, jb.y, jb.n, r + 1, wave, lane);
                load_run(wn, mat, R, C, rows[1], r, h);
            } else if (r + 1 < nr) {
                load_run(wn, mat, R, C, rows[0], r + 1, h);
            }
            mma_run<TYPE, NT>(w, xb, nn, h, acc[g]);
            w = wn;
        }
    }
    if (gu) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int m = 32 * t + 8 * (q / 4) + 4 * h + q % 4;
                if (m < jb.n) {
                    const size_t o = (size_t) jb.out[m];
                    gu[o * R + rows[0]] = acc[0][t][q];
                    gu[o * R + rows[1]] = acc[1][t][q];
                }
            }
    }
    if (h16) {
        // h through LDS ([token][256 FF indices], the last run's buffer is free once every wavefront is past it), then
        // 16-byte stores of whole 512-byte row pieces
        constexpr int HLD = MM_BM + 8;
        _Float16* hs = xs;
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int m = 32 * t + 8 * (q / 4) + 4 * h + q % 4;
                hs[m * HLD + wave * 32 + nn] = (_Float16) (silu_f(acc[0][t][q]) * acc[1][t][q]);
            }
        __syncthreads();
        for (int i = threadIdx.x; i < jb.n * (MM_BM / 8); i += MM_THREADS) {
            const int m = i / (MM_BM / 8), c = i % (MM_BM / 8);
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
    xcd_job(blockIdx.x, ff / MM_BM, sl, ji);
    if (ji >= *njobs) return;
    __shared__ sfnx_bigjob jb;
    extern __shared__ __align__(16) unsigned char xs_raw[];
    load_job(jb, jobs + ji);
    __syncthreads();
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const uint8_t* mat = A + (size_t) jb.w * sa;
    _Float16* xs = reinterpret_cast<_Float16*>(xs_raw);
    if (jb.n > 32) mma_gu_job<TYPE, 2>(mat, ff, C, sl * MM_BM, wave, lane, jb, x, xs, gu, h16);
    else mma_gu_job<TYPE, 1>(mat, ff, C, sl * MM_BM, wave, lane, jb, x, xs, gu, h16);
}

template <int TYPE>
__global__ void __launch_bounds__(MM_THREADS) k_moe_mma(const uint8_t* __restrict__ A, size_t sa, int R, int C, int G,
                                                       const sfnx_bigjob* __restrict__ jobs, const int* __restrict__ njobs,
                                                       const _Float16* __restrict__ x, float* __restrict__ out) {
    int sl, ji;
    xcd_job(blockIdx.x, R / (G * MM_BM), sl, ji);
    const int pj = sl == 0 && ji < 512 ? ji : -1;
    MPROF(0)
    if (ji >= *njobs) return;
    __shared__ sfnx_bigjob jb;
    extern __shared__ __align__(16) unsigned char xs_raw[];
    load_job(jb, jobs + ji);
    __syncthreads();
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const uint8_t* mat = A + (size_t) jb.w * sa;
    _Float16* xs = reinterpret_cast<_Float16*>(xs_raw);
    const int row0 = sl * G * MM_BM;
    MPROF(1)
    if (jb.n > 32) mma_job<TYPE, 2>(mat, R, C, row0, G, wave, lane, jb.y, jb.out, jb.n, x, C, xs, out, pj);
    else mma_job<TYPE, 1>(mat, R, C, row0, G, wave, lane, jb.y, jb.out, jb.n, x, C, xs, out, pj);
    MPROF(18)
}

// k_swiglu_h16 (src/moe_mma.cuh:382-388): h16 = f16(silu(gate) * up) of P rows [gate (ff) | up (ff)]
__global__ void k_swiglu_h16(const float* __restrict__ gu, int ff, int P, _Float16* __restrict__ h16) {
    const size_t n = (size_t) P * ff;
    for (size_t e = blockIdx.x * (size_t) blockDim.x + threadIdx.x; e < n; e += (size_t) gridDim.x * blockDim.x) {
        const size_t p = e / ff, i = e % ff;
        h16[e] = (_Float16) (silu_f(gu[p * 2 * ff + i]) * gu[p * 2 * ff + ff + i]);
    }
}

__global__ void k_to_f16(const float* __restrict__ x, _Float16* __restrict__ y, size_t n) {
    for (size_t e = blockIdx.x * (size_t) blockDim.x + threadIdx.x; e < n; e += (size_t) gridDim.x * blockDim.x)
        y[e] = (_Float16) x[e];
}

constexpr size_t MM_LDS = 2 * MM_XBUF * sizeof(_Float16);

void moe_mma(uint32_t type, const void* A, size_t sa, int n_in, int n_out, const sfnx_bigjob* jobs, const int* njobs,
             int njobs_cap, const void* x16, float* out, void* st) {
    require(type == SFNX_Q4_K || type == SFNX_Q8_0, "expert type must be Q4_K (12) or Q8_0 (8)");
    require(n_in > 0 && n_in % 512 == 0, "expert input width must be a multiple of 512");
    require(n_out > 0 && n_out % MM_BM == 0, "expert rows must be a multiple of 256");
    require((n_out / MM_BM) % std::max(1, (n_out / MM_BM) / 2) == 0, "row groups must split evenly");
    require(sa >= row_bytes(type, n_in) * (size_t) n_out, "expert stride smaller than a matrix");
    require(njobs_cap >= 0 && njobs_cap <= (1 << 20), "njobs_cap out of range");
    if (njobs_cap == 0) return;
    // groups of 256 rows a block: every row in one block when one run covers the input (the activations are staged
    // once); else two blocks a job, for more blocks than compute units
    const int groups = n_out / MM_BM, G = n_in == MM_RUN ? groups : std::max(1, groups / 2);
    const dim3 grid(xcd_grid(groups / G, njobs_cap));
    hipStream_t s = stream_of(st);
    if (type == SFNX_Q4_K)
        k_moe_mma<SFNX_Q4_K><<<grid, MM_THREADS, MM_LDS, s>>>((const uint8_t*) A, sa, n_out, n_in, G, jobs, njobs, (const _Float16*) x16, out);
    else
        k_moe_mma<SFNX_Q8_0><<<grid, MM_THREADS, MM_LDS, s>>>((const uint8_t*) A, sa, n_out, n_in, G, jobs, njobs, (const _Float16*) x16, out);
}

void moe_mma_gu(uint32_t type, const void* A, size_t sa, int n_in, int ff, const sfnx_bigjob* jobs, const int* njobs,
                int njobs_cap, const void* x16, float* gu, uint16_t* h16, void* st) {
    require(type == SFNX_Q4_K || type == SFNX_Q8_0, "expert type must be Q4_K (12) or Q8_0 (8)");
    require(n_in > 0 && n_in % 512 == 0, "expert input width must be a multiple of 512");
    require(ff > 0 && ff % MM_BM == 0, "FF must be a multiple of 256");
    require(sa >= row_bytes(type, n_in) * (size_t) (2 * ff), "expert stride smaller than a matrix");
    require(njobs_cap >= 0 && njobs_cap <= (1 << 20), "njobs_cap out of range");
    if (njobs_cap == 0) return;
    const dim3 grid(xcd_grid(ff / MM_BM, njobs_cap));
    hipStream_t s = stream_of(st);
    if (type == SFNX_Q4_K)
        k_moe_mma_gu<SFNX_Q4_K><<<grid, MM_THREADS, MM_LDS, s>>>((const uint8_t*) A, sa, ff, n_in, jobs, njobs,
                                                                  (const _Float16*) x16, gu, (_Float16*) h16);
    else
        k_moe_mma_gu<SFNX_Q8_0><<<grid, MM_THREADS, MM_LDS, s>>>((const uint8_t*) A, sa, ff, n_in, jobs, njobs,
                                                                  (const _Float16*) x16, gu, (_Float16*) h16);
}

}  // namespace
}  // namespace sfnx

using namespace sfnx;

#ifdef SFNX_PHASE_PROF
extern "C" int sfnx_mma_prof_read(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_mma_prof), sizeof(g_mma_prof)) == hipSuccess ? 0 : -1;
}
#endif

extern "C" int sfnx_moe_gate_up_mma(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_bigjob* jobs,
                                    const int* njobs, int njobs_cap, const uint16_t* xh, float* gu, void* st) {
    return guarded("sfnx_moe_gate_up_mma", [&] {
        if (n_out % (2 * MM_BM) == 0 && n_in > MM_RUN)
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
