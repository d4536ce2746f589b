// Activations and routing: q8_1 quantization, the decode router (logits, top-k, jobs in one launch), the prompt path's
// router logits and permutation, and the weighted combine.
#include "cache.hpp"
#include "topk.hpp"

namespace sfnx {
namespace {

// ------------------------------------------------------------------------------------------------ q8_1
// k_quantize (src/kernels.cu:99-113): a 32-value block per half-wave; d = amax / 127, q = roundf(x / d), ds = {d, sum},
// the sum a xor butterfly 16, 8, 4, 2, 1 (the reference warp's order, kept inside each half of the wave)
__global__ void __launch_bounds__(256) k_quantize_q8_1(const float* __restrict__ x, uint8_t* __restrict__ q, int n, int rows) {
    const int nb = n / 32, row = blockIdx.y, b = blockIdx.x * 8 + (threadIdx.x >> 5), l = threadIdx.x & 31;
    const bool live = b < nb;
    const float xi = live ? x[(size_t) row * n + 32 * b + l] : 0.f;
    const float amax = group_max<32>(fabsf(xi)), sum = group_sum<32>(xi);
    if (!live) return;
    const float d = amax / 127.0f;
    uint8_t* blk = q + ((size_t) row * nb + b) * Q81_BYTES;
    blk[4 + l] = (uint8_t) (int8_t) (amax == 0.0f ? 0 : (int) roundf(xi / d));
    if (l == 0) {
        const uint32_t ds = (uint32_t) f2h(d) | ((uint32_t) f2h(sum) << 16);
        *reinterpret_cast<uint32_t*>(blk) = ds;
    }
}

// ------------------------------------------------------------------------------------------------ router logits
// one wavefront per row: lane l holds the row's float4 chunks l, l + 64, ... (NC of them); per token an fmaf chain
// over those chunks, then a xor butterfly 32 .. 1
template <int NC>
__device__ __forceinline__ void row_load(const float* __restrict__ w, int lane, float4 (&wv)[NC]) {
#pragma unroll
    for (int i = 0; i < NC; ++i) wv[i] = reinterpret_cast<const float4*>(w)[i * WAVE + lane];
}
template <int NC>
__device__ __forceinline__ float row_dot(const float4 (&wv)[NC], const float* __restrict__ x, int lane) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const float4 b = reinterpret_cast<const float4*>(x)[i * WAVE + lane];
        a = fmaf(wv[i].x, b.x, a);
        a = fmaf(wv[i].y, b.y, a);
        a = fmaf(wv[i].z, b.z, a);
        a = fmaf(wv[i].w, b.w, a);
    }
    return group_sum<WAVE>(a);
}

constexpr int RR_THREADS = 256, RR_WAVES = RR_THREADS / WAVE;
// src/moe.cuh:73-202 k_router_route: the router's rows a wavefront each, the shared gate row E included; the last
// block to finish takes the top-K of every token and builds the jobs (first-pick order, rows in pair order).  Returns
// the job count in the last block, -1 in the others.
template <int NC, int TT>
__device__ __forceinline__ int router_route_body(const float* __restrict__ W, const float* __restrict__ x,
                                                 float* __restrict__ logits, int T, int E, int K, int* __restrict__ topi,
                                                 float* __restrict__ topw, sfnx_job* __restrict__ gu,
                                                 sfnx_job* __restrict__ dn, int* __restrict__ njobs, int shared) {
    constexpr int H = NC * 4 * WAVE;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, L = E + 1;
    const int row = blockIdx.x * RR_WAVES + wave;
    if (row < L) {
        float4 wv[NC];
        row_load<NC>(W + (size_t) row * H, lane, wv);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            if (t >= T) break;
            const float s = row_dot<NC>(wv, x + (size_t) t * H, lane);
            if (lane == 0) logits[(size_t) t * L + row] = s;
        }
    }
    __shared__ int last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(njobs + 1, 1) == (int) gridDim.x - 1;
    __syncthreads();
    if (!last) return -1;
    __threadfence();
    __shared__ int ex[MAX_P];
    for (int t = wave; t < T; t += RR_WAVES) {
        int pick;
        float w;
        topk_wave_e<true>(logits + (size_t) t * L, E, K, lane, pick, w);
        if (lane < K) {
            topi[t * K + lane] = pick;
            topw[t * K + lane] = w;
            ex[t * K + lane] = pick;
        }
    }
    __syncthreads();
    // jobs: a job per distinct expert in first-pick order, rows in pair order
    const int P = T * K;
    __shared__ unsigned rows[MAX_E];
    __shared__ int jobof[MAX_E], wsum[MAX_P / WAVE];
    PickSlot ps;
    const int nr = pick_slots(ex, P, K, rows, jobof, wsum, ps);
    const int p = threadIdx.x;
    if (p < P && ps.e >= 0) {
        const int j = ps.job;
        if (ps.slot == 0) {
            gu[j].w = dn[j].w = ps.e;
            gu[j].n = dn[j].n = ps.cnt;
        }
        gu[j].y[ps.slot] = p / K;
        gu[j].out[ps.slot] = dn[j].y[ps.slot] = dn[j].out[ps.slot] = p;
    }
    const int nj = nr;
    if (shared) {
        if (p == 0) {
            gu[nj].w = dn[nj].w = E;
            gu[nj].n = dn[nj].n = T;
        }
        if (p < T) {
            gu[nj].y[p] = p;
            gu[nj].out[p] = dn[nj].y[p] = dn[nj].out[p] = P + p;
        }
    }
    if (p == 0) {
        njobs[0] = nj + (shared ? 1 : 0);
        njobs[1] = 0;
    }
    return nj + (shared ? 1 : 0);
}

template <int NC, int TT>
__global__ void __launch_bounds__(RR_THREADS) k_router_route(const float* __restrict__ W, const float* __restrict__ x,
                                                            float* __restrict__ logits, int T, int E, int K,
                                                            int* __restrict__ topi, float* __restrict__ topw,
                                                            sfnx_job* __restrict__ gu, sfnx_job* __restrict__ dn,
                                                            int* __restrict__ njobs, int shared) {
    router_route_body<NC, TT>(W, x, logits, T, E, K, topi, topw, gu, dn, njobs, shared);
}

// The same with an expert cache: the last block's first wavefront then plans the window's slots for `layer`
// (src/moe.cuh:128-198: the reference's router plans in its last block too), once the block's jobs are written, so a
// cached layer takes no launch of its own for the plan.
template <int NC, int TT>
__global__ void __launch_bounds__(RR_THREADS) k_router_route_plan(const float* __restrict__ W, const float* __restrict__ x,
                                                                 float* __restrict__ logits, int T, int E, int K,
                                                                 int* __restrict__ topi, float* __restrict__ topw,
                                                                 sfnx_job* __restrict__ gu, sfnx_job* __restrict__ dn,
                                                                 int* __restrict__ njobs, int shared,
                                                                 sfnx_expert_cache ec, int layer, int* __restrict__ list) {
    const int nj = router_route_body<NC, TT>(W, x, logits, T, E, K, topi, topw, gu, dn, njobs, shared);
    if (nj < 0) return;
    __syncthreads();   // every job of the block written
    if (threadIdx.x >= WAVE) return;
    plan_window(gu, nj, layer, ec, list, threadIdx.x, WaveSync{});
}

// The xor butterfly of group_sum<64> applied to NV partial sums a lane at once, by recursive halving: at the level of
// lane bit b a lane keeps the half of its values selected by that bit and adds its partner's copy of them, so each
// value meets exactly the partners (and tree) group_sum would give it.  Lane l ends with value l >> (6 - log2 NV), in
// every lane of its group of 64 / NV.
template <int O, int N> __device__ __forceinline__ void halve(float (&v)[N], int n, int lane) {
    const bool up = lane & O;
#pragma unroll
    for (int j = 0; j < N / 2; ++j)
        if (j < n / 2) {
            const float lo = v[j], hi = v[j + n / 2];
            v[j] = (up ? hi : lo) + lane_xor<O>(up ? lo : hi);
        }
}
template <int NV> __device__ __forceinline__ float reduce_scatter(float (&v)[NV], int lane) {
    int n = NV;
    if (n > 1) { halve<32>(v, n, lane); n /= 2; } else v[0] += lane_xor<32>(v[0]);
    if (n > 1) { halve<16>(v, n, lane); n /= 2; } else v[0] += lane_xor<16>(v[0]);
    if (n > 1) { halve<8>(v, n, lane); n /= 2; } else v[0] += lane_xor<8>(v[0]);
    if (n > 1) { halve<4>(v, n, lane); n /= 2; } else v[0] += lane_xor<4>(v[0]);
    if (n > 1) { halve<2>(v, n, lane); n /= 2; } else v[0] += lane_xor<2>(v[0]);
    if (n > 1) { halve<1>(v, n, lane); n /= 2; } else v[0] += lane_xor<1>(v[0]);
    return v[0];
}

// Prompt-path router logits [T][L] = W x for chunks under RM_MIN_T tokens, each (token, row) with row_dot's arithmetic (lane l's fmaf chain over its
// float4 chunks l + 64 i, then the xor butterfly), register-blocked: a wavefront keeps RT router rows in registers and
// takes the block's tokens LT_RU at a time from LDS, where the block stages them by asynchronous global -> LDS copies
// into LT_NBUF buffers (LT_NBUF - 1 groups in flight while one computes); the RT x LT_RU sums of a lane leave through
// one reduce_scatter.  A block: 8 wavefronts of RT rows, and as many tokens as give one block a compute unit.
constexpr int LT_THREADS = 512, LT_WAVES = LT_THREADS / WAVE, LT_RU = 4;
// 3 buffers, 2 past H = 2560 (3 x 4 rows of 4096 floats would pass the 160 KB of LDS a workgroup has)
__host__ __device__ constexpr int lt_nbuf(int NC) { return NC <= 10 ? 3 : 2; }
template <int NC>
__global__ void __launch_bounds__(LT_THREADS) k_router_logits(const float* __restrict__ W, const float* __restrict__ x,
                                                             float* __restrict__ logits, int T, int L, int tok) {
    constexpr int H = NC * 4 * WAVE, RT = NC <= 8 ? 4 : 2, NV = RT * LT_RU, LT_NBUF = lt_nbuf(NC);
    constexpr int PER = LT_RU * H / 4, COPIES = PER / LT_THREADS;   // float4 a group; copies a wavefront issues a group
    static_assert(PER % LT_THREADS == 0, "a group is whole copies");
    extern __shared__ __align__(16) unsigned char lds[];
    float* xs = reinterpret_cast<float*>(lds);   // [LT_NBUF][LT_RU][H]
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int row0 = (blockIdx.x * LT_WAVES + wave) * RT, t0 = blockIdx.y * tok, nt = min(tok, T - t0);
    const int ng = (nt + LT_RU - 1) / LT_RU;
    // group g's LT_RU token rows into buffer g % LT_NBUF (tokens past the end repeat the last); a wavefront moves 64
    // float4 a copy
    auto stage = [&](int g) {
#pragma unroll
        for (int k = 0; k < COPIES; ++k) {
            const int c = (k * LT_WAVES + wave) * WAVE, u = c / (H / 4), col = c % (H / 4);
            const int t = t0 + min(g * LT_RU + u, nt - 1);
            lds_copy_async<16>(x + (size_t) t * H + 4 * (col + lane), xs + (size_t) ((g % LT_NBUF) * LT_RU + u) * H + 4 * col);
        }
    };
    float4 wv[RT][NC];
#pragma unroll
    for (int q = 0; q < RT; ++q) row_load<NC>(W + (size_t) min(row0 + q, L - 1) * H, lane, wv[q]);
    for (int g = 0; g < LT_NBUF - 1; ++g)
        if (g < ng) stage(g);
    for (int g = 0; g < ng; ++g) {
        // group g's copies landed: the ones issued after it (groups g + 1 .. g + LT_NBUF - 2) may still be in flight
        // (the logits stores issued since only make this wait longer).  The barrier has no memory fence, which would
        // wait for those too: every wavefront's copies of group g landed; every wavefront is past group g - 1, whose
        // buffer refills
        if (g + LT_NBUF - 2 < ng) vm_wait<COPIES * (LT_NBUF - 2)>();
        else vm_wait<0>();
        lds_barrier();
        if (g + LT_NBUF - 1 < ng) stage(g + LT_NBUF - 1);
        const float4* xb = reinterpret_cast<const float4*>(xs + (size_t) (g % LT_NBUF) * LT_RU * H);
        float acc[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) acc[k] = 0.f;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            float4 xv[LT_RU];
#pragma unroll
            for (int u = 0; u < LT_RU; ++u) xv[u] = xb[u * (H / 4) + i * WAVE + lane];
#pragma unroll
            for (int q = 0; q < RT; ++q)
#pragma unroll
                for (int u = 0; u < LT_RU; ++u) {
                    float& a = acc[q * LT_RU + u];
                    a = fmaf(wv[q][i].x, xv[u].x, a);
                    a = fmaf(wv[q][i].y, xv[u].y, a);
                    a = fmaf(wv[q][i].z, xv[u].z, a);
                    a = fmaf(wv[q][i].w, xv[u].w, a);
                }
        }
        const float v = reduce_scatter<NV>(acc, lane);
        constexpr int SH = NV == 16 ? 2 : NV == 8 ? 3 : 4;   // lane l holds value l >> SH
        const int k = lane >> SH, q = k / LT_RU, u = k % LT_RU, t = g * LT_RU + u;
        if ((lane & ((1 << SH) - 1)) == 0 && row0 + q < L && t < nt) logits[(size_t) (t0 + t) * L + row0 + q] = v;
    }
}

// The prompt path's router logits [T][L] = W x (src/prefill.cu:1163, the engine's sgemm) on the fp32 matrix cores, for
// chunks of RM_MIN_T tokens or more (fewer leave most compute units idle; they take k_router_logits above).
// v_mfma_f32_16x16x4_f32 adds its 4 k-slots to the accumulator as fmaf in slot order (measured bit for bit on gfx950),
// so a chain of them is an fmaf chain whose order the CPU restatement can follow exactly.  A workgroup owns TOK tokens
// (32, 48, 64 or 96: TOK / 16 tiles of 16) x 48 router rows (3 tiles of 16: 513 rows pad to 528, 11 row tiles);
// its 8 wavefronts split the hidden dimension into 8 slices of H / 8.  A wavefront's lane (m, g) = (lane % 16,
// lane / 16) takes the float4 at column 16 j + 4 g of its token row and of its router row, so MFMA i of step j sums
// columns 16 j + 4 g + i over g = 0..3.  The 8 slices' sums are added in slice order.  Rows past L and tokens past T
// repeat the last one and are not stored.
constexpr int RM_MIN_T = 512;
constexpr int RM_WAVES = 8, RM_THREADS = RM_WAVES * WAVE, RM_RT = 3, RM_ROWS = 16 * RM_RT;
constexpr int RM_PITCH = RM_ROWS + 1, RM_SLOTS = 2;
typedef float float4v __attribute__((ext_vector_type(4)));
// xh (may be null): x as f16 (round to nearest even) as well, written by the workgroups of the first row tile, whose
// wavefronts between them read every value of their tokens' rows once
template <int TOK>
__global__ void __launch_bounds__(RM_THREADS) k_router_mm(const float* __restrict__ W, const float* __restrict__ x,
                                                         float* __restrict__ logits, int T, int H, int L,
                                                         _Float16* __restrict__ xh) {
    constexpr int TU = TOK / 16;
    extern __shared__ __align__(16) unsigned char lds[];
    float* part = reinterpret_cast<float*>(lds);   // [RM_WAVES / 2][TOK][RM_PITCH]
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, m = lane % 16, g = lane / 16;
    const int r0 = blockIdx.x * RM_ROWS, t0 = blockIdx.y * TOK, KW = H / RM_WAVES, k0 = wave * KW + 4 * g;
    const float4v* xa[TU];
    const float4v* wb[RM_RT];
#pragma unroll
    for (int u = 0; u < TU; ++u) xa[u] = reinterpret_cast<const float4v*>(x + (size_t) min(t0 + 16 * u + m, T - 1) * H + k0);
#pragma unroll
    for (int q = 0; q < RM_RT; ++q) wb[q] = reinterpret_cast<const float4v*>(W + (size_t) min(r0 + 16 * q + m, L - 1) * H + k0);
    float4v acc[TU][RM_RT];
#pragma unroll
    for (int u = 0; u < TU; ++u)
#pragma unroll
        for (int q = 0; q < RM_RT; ++q) acc[u][q] = float4v{0.f, 0.f, 0.f, 0.f};
    // Steps of 16 columns, their operands through a ring of RM_SLOTS register slots: step j + RM_SLOTS - 1 is
    // requested when step j starts (the steps a slice has, H / 128, are a multiple of RM_SLOTS)
    const int steps = KW / 16;
    float4v a[RM_SLOTS][TU], b[RM_SLOTS][RM_RT];
    auto request = [&](int slot, int j) {
#pragma unroll
        for (int u = 0; u < TU; ++u) a[slot][u] = xa[u][4 * j];
#pragma unroll
        for (int q = 0; q < RM_RT; ++q) b[slot][q] = wb[q][4 * j];
    };
#pragma unroll
    for (int sl = 0; sl < RM_SLOTS - 1; ++sl) request(sl, sl);
    for (int j0 = 0; j0 < steps; j0 += RM_SLOTS) {
#pragma unroll
        for (int sl = 0; sl < RM_SLOTS; ++sl) {
            const int j = j0 + sl;
            request((sl + RM_SLOTS - 1) % RM_SLOTS, min(j + RM_SLOTS - 1, steps - 1));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int u = 0; u < TU; ++u)
#pragma unroll
                    for (int q = 0; q < RM_RT; ++q)
                        acc[u][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[sl][u][i], b[sl][q][i], acc[u][q], 0, 0, 0);
            if (xh != nullptr && blockIdx.x == 0)
#pragma unroll
                for (int u = 0; u < TU; ++u)
                    if (t0 + 16 * u + m < T) {
                        typedef _Float16 half4v __attribute__((ext_vector_type(4)));
                        const half4v hv = {(_Float16) a[sl][u][0], (_Float16) a[sl][u][1], (_Float16) a[sl][u][2], (_Float16) a[sl][u][3]};
                        *reinterpret_cast<half4v*>(xh + (size_t) (t0 + 16 * u + m) * H + k0 + 16 * j) = hv;
                    }
        }
    }
    // The slices' sums meet in LDS in two halves (half the LDS, so three workgroups share a compute unit): slices 0-3,
    // then 4-7, each output's sum running through them in slice order.  Accumulator element i of tile (u, q) is token
    // 16 u + 4 g + i, router row 16 q + m.
    constexpr int PER = (TOK * RM_ROWS + RM_THREADS - 1) / RM_THREADS;   // outputs a thread sums
    float sum[PER];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        if (wave / (RM_WAVES / 2) == half)
#pragma unroll
            for (int u = 0; u < TU; ++u)
#pragma unroll
                for (int q = 0; q < RM_RT; ++q)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        part[((wave % (RM_WAVES / 2)) * TOK + 16 * u + 4 * g + i) * RM_PITCH + 16 * q + m] = acc[u][q][i];
        __syncthreads();
#pragma unroll
        for (int c = 0; c < PER; ++c) {
            const int o = threadIdx.x + c * RM_THREADS, t = o / RM_ROWS, r = o % RM_ROWS;
            if (o >= TOK * RM_ROWS) break;
#pragma unroll
            for (int w = 0; w < RM_WAVES / 2; ++w) {
                const float p = part[(w * TOK + t) * RM_PITCH + r];
                sum[c] = half == 0 && w == 0 ? p : sum[c] + p;
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int c = 0; c < PER; ++c) {
        const int o = threadIdx.x + c * RM_THREADS, t = o / RM_ROWS, r = o % RM_ROWS;
        if (o < TOK * RM_ROWS && t0 + t < T && r0 + r < L) logits[(size_t) (t0 + t) * L + r0 + r] = sum[c];
    }
}

// ------------------------------------------------------------------------------------------------ prompt routing
// src/prefill.cu:191-221 k_pf_top10: a wavefront per token (the picks are counted by k_pf_fill)
__global__ void __launch_bounds__(RR_THREADS) k_pf_topk(const float* __restrict__ logits, int C, int E, int K,
                                                       int* __restrict__ topi, float* __restrict__ topw) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, t = blockIdx.x * RR_WAVES + wave;
    if (t >= C) return;
    int pick;
    float w;
    topk_wave_e(logits + (size_t) t * (E + 1), E, K, lane, pick, w);
    if (lane < K) {
        topi[(size_t) t * K + lane] = pick;
        topw[(size_t) t * K + lane] = w;
    }
}
// src/prefill.cu:248-279 k_pf_fill: a block per expert ranks its pairs in index order, 4 consecutive pairs a thread and
// 4,096 a pass, its slots from a prefix over the threads of the pass (ballots of the count bits, then the wavefronts in
// order), so a pair always lands in the same job and slot.  The same scan counts every expert's picks in LDS
// (src/prefill.cu:223-226 k_pf_count; block e writes cnt[e]: no global atomics, which serialised on the experts many
// tokens pick); then the block finds its expert's first job (src/prefill.cu:228-242 k_pf_jobbase: the exclusive prefix
// of ceil(cnt / 64) in expert order) and writes the jobs from its ranked list, a pair a thread (a second scan places
// them when more than PF_OWN_MAX tokens pick the expert).  Block 0 writes the job count, and the blocks together lay
// out the shared expert's jobs after the routed ones (tokens in order, 64 a job).
constexpr int PF_FILL_THREADS = 1024, PF_FILL_PASS = 4 * PF_FILL_THREADS, PF_OWN_MAX = 4096;
__global__ void __launch_bounds__(PF_FILL_THREADS) k_pf_fill(const int* __restrict__ topi, int P, int K, int E, int C,
                                                            int shared, int* __restrict__ cnt, int* __restrict__ jbase,
                                                            int* __restrict__ njobs, sfnx_bigjob* __restrict__ gu,
                                                            sfnx_bigjob* __restrict__ dn) {
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int e = blockIdx.x;
    __shared__ int wsum[2][PF_FILL_THREADS / WAVE];
    __shared__ int hist[MAX_E];
    for (int i = tid; i < E; i += PF_FILL_THREADS) hist[i] = 0;
    __syncthreads();
    // one scan: every pair counted, and this expert's pairs ranked in index order (ballot prefixes within a
    // wavefront, then the wavefronts in order) into `own`
    __shared__ int own[PF_OWN_MAX];
    __shared__ int wc1[2][PF_FILL_THREADS / WAVE];
    const uint64_t lt1 = (1ull << lane) - 1ull;
    // a pass's 4 pairs a thread (P is a multiple of 4 or the tail is scalar); the next pass's are requested before
    // this pass's barrier
    auto pairs_at = [&](int p) {
        if (p + 3 < P) return *reinterpret_cast<const int4*>(topi + p);
        return make_int4(p < P ? topi[p] : -1, p + 1 < P ? topi[p + 1] : -1, p + 2 < P ? topi[p + 2] : -1, -1);
    };
    int ce = 0;
    int4 nxt = pairs_at(4 * tid);
    for (int p0 = 0, it = 0; p0 < P; p0 += PF_FILL_PASS, ++it) {
        const int p = p0 + 4 * tid;
        const int q[4] = {nxt.x, nxt.y, nxt.z, nxt.w};
        if (p0 + PF_FILL_PASS < P) nxt = pairs_at(p + PF_FILL_PASS);
        int mine = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (q[c] >= 0) atomicAdd(&hist[q[c]], 1);
            mine += q[c] == e;
        }
        const uint64_t b0 = __ballot(mine & 1), b1 = __ballot(mine & 2), b2 = __ballot(mine & 4);
        if (lane == 0) wc1[it & 1][wave] = __popcll(b0) + 2 * __popcll(b1) + 4 * __popcll(b2);
        __syncthreads();
        int before = __popcll(b0 & lt1) + 2 * __popcll(b1 & lt1) + 4 * __popcll(b2 & lt1), total = 0;
#pragma unroll
        for (int w = 0; w < PF_FILL_THREADS / WAVE; ++w) {
            before += w < wave ? wc1[it & 1][w] : 0;
            total += wc1[it & 1][w];
        }
        int r = ce + before;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (q[c] == e) {
                if (r < PF_OWN_MAX) own[r] = p + c;
                ++r;
            }
        ce += total;
    }
    __syncthreads();
    int jb0 = 0, jall = 0;   // jobs of the experts before e, of all experts
    for (int i = tid; i < E; i += PF_FILL_THREADS) {
        const int nj = (hist[i] + SFNX_PF_JOB - 1) / SFNX_PF_JOB;
        jb0 += i < e ? nj : 0;
        jall += nj;
    }
    jb0 = group_isum<WAVE>(jb0);
    jall = group_isum<WAVE>(jall);
    if (lane == 0) {
        wsum[0][wave] = jb0;
        wsum[1][wave] = jall;
    }
    __syncthreads();
    jb0 = jall = 0;
#pragma unroll
    for (int w = 0; w < PF_FILL_THREADS / WAVE; ++w) {
        jb0 += wsum[0][w];
        jall += wsum[1][w];
    }
    if (shared) {   // the shared expert's jobs, its tokens spread over the blocks
        for (int t = e * PF_FILL_THREADS + tid; t < C; t += E * PF_FILL_THREADS) {
            const int j = jall + t / SFNX_PF_JOB, k = t % SFNX_PF_JOB;
            gu[j].y[k] = t;
            gu[j].out[k] = dn[j].y[k] = dn[j].out[k] = P + t;
            if (k == 0) {
                gu[j].w = dn[j].w = E;
                gu[j].n = dn[j].n = min(SFNX_PF_JOB, C - t);
            }
        }
    }
    if (tid == 0) {
        cnt[e] = ce;
        jbase[e] = jb0;
        if (e == 0) njobs[0] = jall + (shared ? (C + SFNX_PF_JOB - 1) / SFNX_PF_JOB : 0);
    }
    if (ce == 0) return;
    if (ce <= PF_OWN_MAX) {   // the jobs straight from the ranked list, a pair a thread
        for (int r = tid; r < ce; r += PF_FILL_THREADS) {
            const int pc = own[r], j = jb0 + r / SFNX_PF_JOB, k = r % SFNX_PF_JOB;
            gu[j].y[k] = pc / K;
            gu[j].out[k] = pc;
            dn[j].y[k] = pc;
            dn[j].out[k] = pc;
            if (k == 0) {
                gu[j].w = dn[j].w = e;
                gu[j].n = dn[j].n = min(SFNX_PF_JOB, ce - r);
            }
        }
        return;
    }
    // more pairs than the list holds: a second scan places them
    __shared__ int wcount[2][PF_FILL_THREADS / WAVE];
    const uint64_t lt = (1ull << lane) - 1ull;
    int base = 0;
    for (int p0 = 0, it = 0; p0 < P; p0 += PF_FILL_PASS, ++it) {
        const int p = p0 + 4 * tid;
        int q[4];
        if (p + 3 < P) {
            const int4 v = *reinterpret_cast<const int4*>(topi + p);   // P is a multiple of 4 or the tail is scalar
            q[0] = v.x, q[1] = v.y, q[2] = v.z, q[3] = v.w;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) q[c] = p + c < P ? topi[p + c] : -1;
        }
        int mine = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) mine += q[c] == e;
        // this thread's exclusive prefix within its wavefront: the count's bits by ballot
        const uint64_t b0 = __ballot(mine & 1), b1 = __ballot(mine & 2), b2 = __ballot(mine & 4);
        const int before_w = __popcll(b0 & lt) + 2 * __popcll(b1 & lt) + 4 * __popcll(b2 & lt);
        const int total_w = __popcll(b0) + 2 * __popcll(b1) + 4 * __popcll(b2);
        if (lane == 0) wcount[it & 1][wave] = total_w;
        __syncthreads();
        int before = before_w, total = 0;
#pragma unroll
        for (int w = 0; w < PF_FILL_THREADS / WAVE; ++w) {
            before += w < wave ? wcount[it & 1][w] : 0;
            total += wcount[it & 1][w];
        }
        int s = base + before;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (q[c] == e) {
                const int pc = p + c, j = jb0 + s / SFNX_PF_JOB, k = s % SFNX_PF_JOB;
                gu[j].y[k] = pc / K;
                gu[j].out[k] = pc;
                dn[j].y[k] = pc;
                dn[j].out[k] = pc;
                if (k == 0) {
                    const int n = min(SFNX_PF_JOB, ce - (s / SFNX_PF_JOB) * SFNX_PF_JOB);
                    gu[j].w = dn[j].w = e;
                    gu[j].n = dn[j].n = n;
                }
                ++s;
            }
        base += total;
    }
}

// ------------------------------------------------------------------------------------------------ combine
// src/kernels.cu:797-803 ring_x / src/prefill.cu:476-484 k_pfr_addend
// The combine (src/kernels.cu:797-803, src/prefill.cu:476-484): y[t][i] = fmaf(sigmoid(l[t][E]), part[T K + t][i],
// sum_k fmaf(w[t][k], part[t K + k][i], .)) in k order, picks of -1 skipped.  A block per (token, 1024 columns): the
// token's picks and weights are wave-uniform, and a thread's 4 columns of every part row are requested before the chain.
constexpr int CB_THREADS = 256;
__global__ void __launch_bounds__(CB_THREADS) k_combine(const float* __restrict__ part, const float* __restrict__ topw,
                                                       const int* __restrict__ topi, const float* __restrict__ logits,
                                                       float* __restrict__ y, int T, int H, int E, int K, int shared) {
    const int t = blockIdx.y, i = (blockIdx.x * CB_THREADS + threadIdx.x) * 4;
    if (i >= H) return;
    float4 pv[MAX_K + 1];
#pragma unroll
    for (int k = 0; k < MAX_K; ++k)
        if (k < K) pv[k] = *reinterpret_cast<const float4*>(part + ((size_t) t * K + k) * H + i);
    if (shared) pv[MAX_K] = *reinterpret_cast<const float4*>(part + ((size_t) T * K + t) * H + i);
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < MAX_K; ++k)
        if (k < K && topi[t * K + k] >= 0) {
            const float w = topw[t * K + k];
            s.x = fmaf(w, pv[k].x, s.x);
            s.y = fmaf(w, pv[k].y, s.y);
            s.z = fmaf(w, pv[k].z, s.z);
            s.w = fmaf(w, pv[k].w, s.w);
        }
    if (shared) {
        const float g = sigm_f(logits[(size_t) t * (E + 1) + E]);
        s.x = fmaf(g, pv[MAX_K].x, s.x);
        s.y = fmaf(g, pv[MAX_K].y, s.y);
        s.z = fmaf(g, pv[MAX_K].z, s.z);
        s.w = fmaf(g, pv[MAX_K].w, s.w);
    }
    *reinterpret_cast<float4*>(y + (size_t) t * H + i) = s;
}

// the stacked-layer driver's glue between MoE layers: x += y, then xn = x / sqrt(mean(x^2) + eps) (an RMSNorm without
// gain, standing in for the engine's hyper-connection read, src/hc.cuh, that normalises the MoE input); a block per
// token, the mean square by one wavefront in the order of wave_rms_scale
constexpr int RN_THREADS = 256;
__global__ void __launch_bounds__(RN_THREADS) k_residual_rmsnorm(float* __restrict__ x, const float* __restrict__ y,
                                                                float* __restrict__ xn, int H, float eps) {
    extern __shared__ __align__(16) float xs[];
    __shared__ float rs;
    const int t = blockIdx.x;
    float* xr = x + (size_t) t * H;
    for (int i = threadIdx.x; i < H; i += RN_THREADS) {
        float v = xr[i];
        if (y) {
            v += y[(size_t) t * H + i];
            xr[i] = v;
        }
        xs[i] = v;
    }
    __syncthreads();
    if (threadIdx.x < WAVE) {
        const float r = wave_rms_scale(xs, H, threadIdx.x, eps);
        if (threadIdx.x == 0) rs = r;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < H; i += RN_THREADS) xn[(size_t) t * H + i] = xs[i] * rs;
}

template <int TT>
void launch_router_tt(int nc, dim3 g, hipStream_t s, const float* W, const float* x, float* logits, int T, int E, int K,
                      int* topi, float* topw, sfnx_job* gu, sfnx_job* dn, int* njobs, int shared) {
    switch (nc) {
        case 4: k_router_route<4, TT><<<g, RR_THREADS, 0, s>>>(W, x, logits, T, E, K, topi, topw, gu, dn, njobs, shared); break;
        case 8: k_router_route<8, TT><<<g, RR_THREADS, 0, s>>>(W, x, logits, T, E, K, topi, topw, gu, dn, njobs, shared); break;
        case 10: k_router_route<10, TT><<<g, RR_THREADS, 0, s>>>(W, x, logits, T, E, K, topi, topw, gu, dn, njobs, shared); break;
        case 16: k_router_route<16, TT><<<g, RR_THREADS, 0, s>>>(W, x, logits, T, E, K, topi, topw, gu, dn, njobs, shared); break;
        default: throw std::runtime_error("hidden size must be 1024, 2048, 2560 or 4096");
    }
}

template <int TT>
void launch_router_plan_tt(int nc, dim3 g, hipStream_t s, const float* W, const float* x, float* logits, int T, int E,
                           int K, int* topi, float* topw, sfnx_job* gu, sfnx_job* dn, int* njobs, int shared,
                           const sfnx_expert_cache& ec, int layer, int* list) {
#define SFNX_RRP(NCV) k_router_route_plan<NCV, TT><<<g, RR_THREADS, 0, s>>>(W, x, logits, T, E, K, topi, topw, gu, dn, njobs, shared, ec, layer, list)
    switch (nc) {
        case 4: SFNX_RRP(4); break;
        case 8: SFNX_RRP(8); break;
        case 10: SFNX_RRP(10); break;
        case 16: SFNX_RRP(16); break;
        default: throw std::runtime_error("hidden size must be 1024, 2048, 2560 or 4096");
    }
#undef SFNX_RRP
}

}  // namespace
}  // namespace sfnx

using namespace sfnx;

extern "C" int sfnx_quantize_q8_1(const float* x, void* q, int n, int rows, void* st) {
    return guarded("sfnx_quantize_q8_1", [&] {
        require(n > 0 && n % 32 == 0, "n must be a positive multiple of 32");
        if (rows <= 0) return;
        require(rows <= 65535, "at most 65535 rows a call");
        k_quantize_q8_1<<<dim3((n / 32 + 7) / 8, rows), 256, 0, stream_of(st)>>>(x, (uint8_t*) q, n, rows);
    });
}

extern "C" int sfnx_router_route(const float* W, const float* x, float* logits, int T, int H, int E, int K, int* topi,
                                 float* topw, sfnx_job* jobs_gu, sfnx_job* jobs_dn, int* njobs, int shared, void* st) {
    return guarded("sfnx_router_route", [&] {
        require(T >= 1 && T <= SFNX_MAXT, "T out of range (1..16)");
        require(E >= WAVE && E % WAVE == 0 && E <= MAX_E, "E must be a multiple of 64, at most 1024");
        require(K >= 1 && K <= MAX_K && K <= E, "K out of range (1..16)");
        require(H % 256 == 0, "H must be a multiple of 256");
        const dim3 g((E + 1 + RR_WAVES - 1) / RR_WAVES);
        const int nc = H / 256;
        hipStream_t s = stream_of(st);
        if (T == 1) launch_router_tt<1>(nc, g, s, W, x, logits, T, E, K, topi, topw, jobs_gu, jobs_dn, njobs, shared);
        else if (T <= 4) launch_router_tt<4>(nc, g, s, W, x, logits, T, E, K, topi, topw, jobs_gu, jobs_dn, njobs, shared);
        else launch_router_tt<16>(nc, g, s, W, x, logits, T, E, K, topi, topw, jobs_gu, jobs_dn, njobs, shared);
    });
}

extern "C" int sfnx_router_route_plan(const float* W, const float* x, float* logits, int T, int H, int E, int K, int* topi,
                                      float* topw, sfnx_job* jobs_gu, sfnx_job* jobs_dn, int* njobs, int shared,
                                      const sfnx_expert_cache* ec, int layer, int* list, void* st) {
    return guarded("sfnx_router_route_plan", [&] {
        require(T >= 1 && T <= SFNX_MAXT, "T out of range (1..16)");
        require(E >= WAVE && E % WAVE == 0 && E <= MAX_E, "E must be a multiple of 64, at most 1024");
        require(K >= 1 && K <= MAX_K && K <= E, "K out of range (1..16)");
        require(H % 256 == 0, "H must be a multiple of 256");
        require(list != nullptr, "null list");
        check_cache(ec);
        check_layer(ec, layer);
        require(E + (shared ? 1 : 0) <= ec->n_experts, "the layer's experts (and its shared expert) pass the cache's tables");
        const dim3 g((E + 1 + RR_WAVES - 1) / RR_WAVES);
        const int nc = H / 256;
        hipStream_t s = stream_of(st);
        if (T == 1) launch_router_plan_tt<1>(nc, g, s, W, x, logits, T, E, K, topi, topw, jobs_gu, jobs_dn, njobs, shared, *ec, layer, list);
        else if (T <= 4) launch_router_plan_tt<4>(nc, g, s, W, x, logits, T, E, K, topi, topw, jobs_gu, jobs_dn, njobs, shared, *ec, layer, list);
        else launch_router_plan_tt<16>(nc, g, s, W, x, logits, T, E, K, topi, topw, jobs_gu, jobs_dn, njobs, shared, *ec, layer, list);
    });
}

// the kernel allowed its dynamic LDS (up to 120 KB) once, then launched
template <int NC>
void launch_logits(dim3 g, hipStream_t s, const float* W, const float* x, float* logits, int T, int L, int tok) {
    const size_t lds = (size_t) lt_nbuf(NC) * LT_RU * NC * 4 * WAVE * 4;
    static const hipError_t allowed =
        hipFuncSetAttribute((const void*) k_router_logits<NC>, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
    check(allowed, "hipFuncSetAttribute");
    k_router_logits<NC><<<g, LT_THREADS, lds, s>>>(W, x, logits, T, L, tok);
}

namespace {
// sfnx_router_logits(_xh): the VALU kernel under RM_MIN_T tokens (xh then by a conversion launch), else k_router_mm
void router_logits(const float* W, const float* x, float* logits, int T, int H, int L, _Float16* xh, hipStream_t st) {
    {
        require(H % 256 == 0, "H must be a multiple of 256");
        if (T <= 0 || L <= 0) return;
        if (T < RM_MIN_T) {   // the VALU kernel (row_dot's order)
            const int rt = H / 256 <= 8 ? 4 : 2, rb = (L + LT_WAVES * rt - 1) / (LT_WAVES * rt);
            // tokens a block (a multiple of LT_RU): the fewest that keep the grid within one block a compute unit
            static const int ncu = [] {
                int n = 0;
                check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, 0), "hipDeviceGetAttribute");
                return n;
            }();
            int tok = LT_RU;
            while ((long) rb * ((T + tok - 1) / tok) > ncu && tok < T) tok += LT_RU;
            const dim3 g(rb, (T + tok - 1) / tok);
            hipStream_t s = st;
            switch (H / 256) {
                case 4: launch_logits<4>(g, s, W, x, logits, T, L, tok); break;
                case 8: launch_logits<8>(g, s, W, x, logits, T, L, tok); break;
                case 10: launch_logits<10>(g, s, W, x, logits, T, L, tok); break;
                case 16: launch_logits<16>(g, s, W, x, logits, T, L, tok); break;
                default: throw std::runtime_error("hidden size must be 1024, 2048, 2560 or 4096");
            }
            check(hipGetLastError(), "k_router_logits launch");
            if (xh) require(sfnx_to_f16(x, (uint16_t*) xh, (size_t) T * H, st) == 0, "sfnx_to_f16 failed");
            return;
        }
        // tokens a workgroup: a taller tile requests fewer operands a multiply-add but makes fewer workgroups.  The
        // estimate: rounds of workgroups over the compute units times a round's time for the tile (measured at 2048
        // columns, the ratios hold for the others: 26, 34, 40, 60 us at 32, 48, 64, 96 tokens)
        static const int ncu = [] {   // once (a static initializer: thread-safe), with the 96-token tile's LDS allowed
            int n = 0;
            check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, 0), "hipDeviceGetAttribute");
            check(hipFuncSetAttribute((const void*) k_router_mm<96>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      RM_WAVES / 2 * 96 * RM_PITCH * 4), "hipFuncSetAttribute");
            return n;
        }();
        const int rb = (L + RM_ROWS - 1) / RM_ROWS;
        int tok = 32;
        long best = 0;
        for (const auto& [tk, round_us] : {std::pair<int, long>{32, 26}, {48, 34}, {64, 40}, {96, 60}}) {
            const long nb = (long) rb * ((T + tk - 1) / tk), cost = (nb + ncu - 1) / ncu * round_us;
            if (tk == 32 || cost < best) tok = tk, best = cost;
        }
        const dim3 g(rb, (T + tok - 1) / tok);
        const size_t lds = (size_t) RM_WAVES / 2 * tok * RM_PITCH * 4;
        switch (tok) {
            case 32: k_router_mm<32><<<g, RM_THREADS, lds, st>>>(W, x, logits, T, H, L, xh); break;
            case 48: k_router_mm<48><<<g, RM_THREADS, lds, st>>>(W, x, logits, T, H, L, xh); break;
            case 64: k_router_mm<64><<<g, RM_THREADS, lds, st>>>(W, x, logits, T, H, L, xh); break;
            default: k_router_mm<96><<<g, RM_THREADS, lds, st>>>(W, x, logits, T, H, L, xh); break;
        }
        check(hipGetLastError(), "k_router_mm launch");
    }
}
}  // namespace

extern "C" int sfnx_router_logits(const float* W, const float* x, float* logits, int T, int H, int L, void* st) {
    return guarded("sfnx_router_logits", [&] { router_logits(W, x, logits, T, H, L, nullptr, stream_of(st)); });
}

extern "C" int sfnx_router_logits_xh(const float* W, const float* x, float* logits, uint16_t* xh, int T, int H, int L,
                                     void* st) {
    return guarded("sfnx_router_logits_xh", [&] {
        require(xh != nullptr, "xh is null");
        router_logits(W, x, logits, T, H, L, reinterpret_cast<_Float16*>(xh), stream_of(st));
    });
}

extern "C" int sfnx_pf_route(const float* logits, int C, int E, int K, int* topi, float* topw, int* cnt, int* jbase,
                             sfnx_bigjob* jobs_gu, sfnx_bigjob* jobs_dn, int* njobs, int shared, void* st) {
    return guarded("sfnx_pf_route", [&] {
        require(C >= 1, "C must be positive");
        require(E >= WAVE && E % WAVE == 0 && E <= MAX_E, "E must be a multiple of 64, at most 1024");
        require(K >= 1 && K <= MAX_K && K <= E, "K out of range (1..16)");
        hipStream_t s = stream_of(st);
        const int P = C * K;
        k_pf_topk<<<(C + RR_WAVES - 1) / RR_WAVES, RR_THREADS, 0, s>>>(logits, C, E, K, topi, topw);
        k_pf_fill<<<E, PF_FILL_THREADS, 0, s>>>(topi, P, K, E, C, shared, cnt, jbase, njobs, jobs_gu, jobs_dn);
    });
}

extern "C" int sfnx_moe_combine(const float* part, const float* topw, const int* topi, const float* logits, float* y, int T,
                                int H, int E, int K, int shared, void* st) {
    return guarded("sfnx_moe_combine", [&] {
        if (T <= 0) return;
        const size_t n = (size_t) T * H;
        require(H % 4 == 0, "H must be a multiple of 4");
        require(K >= 1 && K <= MAX_K, "K out of range (1..16)");
        (void) n;
        const dim3 g((H / 4 + CB_THREADS - 1) / CB_THREADS, T);
        k_combine<<<g, CB_THREADS, 0, stream_of(st)>>>(part, topw, topi, logits, y, T, H, E, K, shared);
    });
}

extern "C" int sfnx_residual_rmsnorm(float* x, const float* y, float* xn, int T, int H, float eps, void* st) {
    return guarded("sfnx_residual_rmsnorm", [&] {
        require(H > 0, "H must be positive");
        if (T <= 0) return;
        require(H > 0 && H % 256 == 0 && H <= 16384, "H must be a multiple of 256, at most 16384");
        k_residual_rmsnorm<<<T, RN_THREADS, H * sizeof(float), stream_of(st)>>>(x, y, xn, H, eps);
    });
}
