// The decode window's MoE layers as three launches each, no atomics and no device-wide fences (a grid barrier costs
// several kernel boundaries on this chip, and an agent-scope fence writes back the whole L2):
//
//   K1 k_dec_router: RMSNorm of the residual stream on the fly, the router's logits (a row a wavefront), and the
//      normalised activations as q8_1 (every block a share of the 32-blocks).
//   K2 k_dec_experts: every block takes the top-K of the logits itself and numbers the jobs (the same deterministic
//      first-pick order as router_route); a block is one unit (job, 32 FF indices): 32 gate rows and the 32 matching up
//      rows dotted with the job's rows, SwiGLU in registers, h quantized to q8_1 per 32 (k_moe_h, src/moe.cuh:284-295).
//   K3 k_dec_down: a block owns 8 output rows: the down rows of every job for those outputs, then the weighted combine
//      in the reference's fmaf order (src/kernels.cu:797-803) and the residual add.
//
// The arithmetic of every value is the unfused entry points' (router_route, moe_gate_up, moe_down, moe_combine), so the
// two paths agree bit for bit.
#include <hip/hip_ext.h>

#include <mutex>

#include "decode.hpp"

namespace sfnx {
namespace {


constexpr int D1_THREADS = 64, D1_WAVES = D1_THREADS / WAVE;   // K1: a router row per wavefront
constexpr int D3_THREADS = 256, D3_ROWS = 8;                    // K3: output rows per block
template <int TYPE> constexpr int d2_threads() { return 32 * lpr_of<TYPE>(); }   // K2: 32 FF indices a block

// ------------------------------------------------------------------------------------------------ K1
// windows: 4 wavefronts a block on the block's row, wavefront g taking tokens g, g + 4, ... (each logit's lanes and
// order as with one wavefront)
template <int TT> constexpr int d1_groups() { return TT > 1 ? 4 : 1; }
template <int NC, int TT>
__global__ void __launch_bounds__(D1_THREADS * d1_groups<TT>()) k_dec_router(const float* __restrict__ W, const float* __restrict__ x, int T,
                                                          int E, float eps, int norm, float* __restrict__ logits,
                                                          uint8_t* __restrict__ xq) {
    constexpr int H = NC * 4 * WAVE, NQ = 2, TG = d1_groups<TT>(), NTH = D1_THREADS * TG;
    static_assert(D1_WAVES == 1, "a router row a block");
    const int tg = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, L = E + 1;
    const int row = blockIdx.x;
    // every load of the launch issued up front: the router row, each token's chunks, this half-wave's q8_1 blocks
    const int nb = H / 32, hw = threadIdx.x / 32, l = threadIdx.x % 32, nslot = gridDim.x * (NTH / 32);
    float xqv[NQ];
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int q = blockIdx.x * (NTH / 32) + hw + k * nslot;
        xqv[k] = q < T * nb ? x[(size_t) (q / nb) * H + 32 * (q % nb) + l] : 0.f;
    }
    const bool live = row < L;
    float4 wv[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) wv[i] = reinterpret_cast<const float4*>(W + (size_t) (live ? row : 0) * H)[i * WAVE + lane];
    __shared__ float rs[SFNX_MAXT];
    // windows: the wavefront's next token's chunks are loaded while this token's reductions run
    float4 xn[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) xn[i] = reinterpret_cast<const float4*>(x + (size_t) min(tg, T - 1) * H)[i * WAVE + lane];
#pragma unroll
    for (int t0 = 0; t0 < TT; t0 += TG) {
        const int t = t0 + tg;
        if (t >= T) break;
        float4 xv[NC];
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NC; ++i) xv[i] = xn[i];
        if (TT > 1 && t + TG < T) {
            const float4* x4 = reinterpret_cast<const float4*>(x + (size_t) (t + TG) * H);
#pragma unroll
            for (int i = 0; i < NC; ++i) xn[i] = x4[i * WAVE + lane];
        }
#pragma unroll
        for (int i = 0; i < NC; ++i) ss = rms_lane_add(xv[i], ss);
        const float r = norm ? rms_from_sum(ss, H, eps) : 1.0f;
        if (lane == 0) rs[t] = r;
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            a = fmaf(wv[i].x, xv[i].x * r, a);
            a = fmaf(wv[i].y, xv[i].y * r, a);
            a = fmaf(wv[i].z, xv[i].z * r, a);
            a = fmaf(wv[i].w, xv[i].w * r, a);
        }
        a = group_sum<WAVE>(a);
        if (live && lane == 0) logits[(size_t) t * L + row] = a;
    }
    __syncthreads();
    // the normalised rows as q8_1 (k_quantize's arithmetic), a half-wave per 32-block, spread over the grid
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int q = blockIdx.x * (NTH / 32) + hw + k * nslot;
        if (q >= T * nb) break;
        const int t = q / nb;
        const float xi = xqv[k] * rs[t];
        const float amax = group_max<32>(fabsf(xi)), sum = group_sum<32>(xi);
        const float d = amax / 127.0f;
        uint8_t* blk = xq + (size_t) q * Q81_BYTES;
        blk[4 + l] = (uint8_t) (int8_t) (amax == 0.0f ? 0 : (int) roundf(xi / d));
        if (l == 0) *reinterpret_cast<uint32_t*>(blk) = (uint32_t) f2h(d) | ((uint32_t) f2h(sum) << 16);
    }
    // small grids: the blocks past the preloaded ones
    for (int q = blockIdx.x * (NTH / 32) + hw + NQ * nslot; q < T * nb; q += nslot) {
        const int t = q / nb;
        const float xi = x[(size_t) t * H + 32 * (q % nb) + l] * rs[t];
        const float amax = group_max<32>(fabsf(xi)), sum = group_sum<32>(xi);
        const float d = amax / 127.0f;
        uint8_t* blk = xq + (size_t) q * Q81_BYTES;
        blk[4 + l] = (uint8_t) (int8_t) (amax == 0.0f ? 0 : (int) roundf(xi / d));
        if (l == 0) *reinterpret_cast<uint32_t*>(blk) = (uint32_t) f2h(d) | ((uint32_t) f2h(sum) << 16);
    }
}

// ------------------------------------------------------------------------------------------------ K2
// K1b for windows of several rows: the routing once (the top-k of every row, a wavefront a row, then the decode job
// numbering of src/moe.cuh:164-198), published for K2, K3 and the caller.  At batch 1, K2's blocks take the top-k
// themselves (k_dec_experts1); with more rows each block would repeat every row's top-k and the numbering.
constexpr int DR_THREADS = 1024;   // a wavefront per row (T <= 16) and a thread per pick
__global__ void __launch_bounds__(DR_THREADS) k_dec_route(int T, int E, int K, int shared, const float* __restrict__ logits,
                                                          int* __restrict__ topi_g, float* __restrict__ topw_g,
                                                          sfnx_job* __restrict__ jg, sfnx_job* __restrict__ jd,
                                                          int* __restrict__ njobs_g) {
    constexpr int NW = DR_THREADS / WAVE;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, p = threadIdx.x, P = T * K;
    __shared__ int ex[MAX_P];
    __shared__ float sw[MAX_P];
    __shared__ unsigned rows[MAX_E];
    __shared__ int jobof[MAX_E], wsum[MAX_P / WAVE];
    for (int t = wave; t < T; t += NW) {
        int pick;
        float w;
        topk_wave_e(logits + (size_t) t * (E + 1), E, K, lane, pick, w);
        if (lane < K) {
            ex[t * K + lane] = pick;
            sw[t * K + lane] = w;
        }
    }
    __syncthreads();
    PickSlot ps;
    const int nr = pick_slots(ex, P, K, rows, jobof, wsum, ps);
    if (p < P) {
        topi_g[p] = ex[p];
        topw_g[p] = sw[p];
        if (ps.e >= 0) {
            const int j = ps.job;
            if (ps.slot == 0) {
                jg[j].w = jd[j].w = ps.e;
                jg[j].n = jd[j].n = ps.cnt;
            }
            jg[j].y[ps.slot] = p / K;
            jg[j].out[ps.slot] = jd[j].y[ps.slot] = jd[j].out[ps.slot] = p;
        }
    }
    if (shared) {
        if (p == 0) {
            jg[nr].w = jd[nr].w = E;
            jg[nr].n = jd[nr].n = T;
        }
        if (p < T) {
            jg[nr].y[p] = p;
            jg[nr].out[p] = jd[nr].y[p] = jd[nr].out[p] = P + p;
        }
    }
    if (p == 0) {
        njobs_g[0] = nr + (shared ? 1 : 0);
        njobs_g[1] = 0;
    }
}

// K2 for windows of several rows: a block is one (job, 32 FF indices) unit of the jobs K1b numbered, as at batch 1:
// the first half of the waves take the 32 gate rows, the second half the matching up rows (a row a lane group, so a
// lane holds one row's share), each dotted with the job's staged activation rows; SwiGLU and h as q8_1 per slot.
template <int TYPE, int G, int TT>
__global__ void __launch_bounds__(2 * d2_threads<TYPE>()) k_dec_experts(
    const uint8_t* __restrict__ A, size_t sa, int H, int E, int ff, const uint8_t* __restrict__ xq,
    const sfnx_job* __restrict__ jg, const int* __restrict__ njobs_g, float* __restrict__ gu, int8_t* __restrict__ hq_q,
    float* __restrict__ hq_d, int* __restrict__ hq_s, Q8sPlanes sh_gu) {
    constexpr int LPR = lpr_of<TYPE>(), NTH = 2 * d2_threads<TYPE>(), NW = NTH / WAVE, RPW = WAVE / LPR;
    const int NFB = ff / 32, fb = blockIdx.x % NFB, nj = njobs_g[0];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    __shared__ sfnx_job jb;
    __shared__ float gbuf[SFNX_MAXT][32], ubuf[SFNX_MAXT][32];
    extern __shared__ __align__(16) unsigned char lds[];
    if ((int) blockIdx.x / NFB >= nj) return;
    // the last job first: with a shared expert it is the shared job, which holds every row of the window and so takes
    // the longest (2.5x a routed job's blocks at 16 rows); dispatched last, its blocks ran alone at the kernel's end
    const int myjob = ((int) blockIdx.x / NFB + nj - 1) % nj;
    load_job(jb, jg + myjob);
    __syncthreads();
    const bool up = wave >= NW / 2;
    const int rw = lane / LPR, ln = lane % LPR, fl = (up ? wave - NW / 2 : wave) * RPW + rw, row = (up ? ff : 0) + fb * 32 + fl;
    auto put = [&](int s, float v) {
        if (ln == 0) {
            gu[(size_t) jb.out[s] * 2 * ff + row] = v;
            (up ? ubuf : gbuf)[s][fl] = v;
        }
    };
    // the weight rows are requested first, then the job's rows of activations staged (slot s holds row jb.y[s]): the
    // two fetches overlap instead of following each other
    const bool dense_sh = sh_gu.q != nullptr && jb.w == E;   // the shared expert's own dense Q8_0 matrix
    typename RowOf<TYPE, G>::R w;
    if (!dense_sh) RowOf<TYPE, G>::load(w, expert_at(A, sa, jb.w), 2 * ff, row, H, ln);
    const Acts a = acts_in(lds, TT, H);
    stage_q8_1(a, xq, jb.y, jb.n);
    __syncthreads();   // the staged activations
    if (dense_sh) {   // the reference's q8s sums
        const Q8sPlanes Ps = sh_gu;
        for (int s = 0; s < jb.n; ++s) put(s, group_sum<LPR>(q8s_dot<LPR>(Ps, row, H, ln, a, s)));
    } else {
        for (int s = 0; s < jb.n; ++s) put(s, group_sum<LPR>(w.dot(a, s, ln)));
    }
    __syncthreads();
    for (int s = threadIdx.x / 32; s < jb.n; s += NTH / 32) {
        const int l = threadIdx.x % 32, o = jb.out[s];
        const float v = silu_f(gbuf[s][l]) * ubuf[s][l];
        const float amax = group_max<32>(fabsf(v));
        const float d = amax / 127.0f;
        const int q = amax == 0.0f ? 0 : (int) roundf(v / d);
        const int qs = group_isum<32>(q);
        hq_q[(size_t) o * ff + 32 * fb + l] = (int8_t) q;
        if (l == 0) {
            hq_d[(size_t) o * NFB + fb] = h2f(f2h(d));
            hq_s[(size_t) o * NFB + fb] = qs;
        }
    }
}

// K1's workgroup b' owns the router rows [D1_WAVES b', D1_WAVES b' + D1_WAVES), on XCD b' % 8.  Workgroup b of a launch
// whose grid is a multiple of 8 warms the next layer's router rows of the K1 workgroups b' = b (mod the grid).
// NTH: the block's threads, a constant (blockDim.x is read from memory, and in this loop the read was repeated and
// waited for, with every warm-up request before it, at each turn)
template <int NTH> __device__ inline void warm_router_rows(const float* W, int rows, int H, void* junk) {
    if (W == nullptr || gridDim.x % XCDS != 0) return;
    const int per_row = H * 4 / LINE, per_blk = D1_WAVES * per_row, nk1 = (rows + D1_WAVES - 1) / D1_WAVES;
    const int mine = (nk1 - (int) blockIdx.x + (int) gridDim.x - 1) / (int) gridDim.x;
    for (int li = threadIdx.x; li < mine * per_blk; li += NTH) {
        const int b1 = blockIdx.x + gridDim.x * (li / per_blk), row = D1_WAVES * b1 + (li % per_blk) / per_row;
        if (row < rows) warm_line(reinterpret_cast<const uint8_t*>(W + (size_t) row * H) + LINE * (li % per_row), junk);
    }
}

// K2 for a window of one row (the batch-1 decode): the picks of one token are distinct experts, so job j is pick j
// (n = 1, row 0, output pair j) and the shared expert's job is the last; no numbering is needed.  Every wavefront takes
// the top-K itself from registers, so the weight loads wait on no barrier after the routing.
// SHQ: a dense Q8_0 shared expert (sh_gu), in an instantiation of its own so the routed-only kernel keeps its registers
template <int TYPE, int G, int NV, bool SHQ>
__global__ void __launch_bounds__(2 * d2_threads<TYPE>()) k_dec_experts1(
    const uint8_t* __restrict__ A, size_t sa, const float* __restrict__ Wn, int H, int E, int K, int ff, int shared,
    const float* __restrict__ logits,
    const uint8_t* __restrict__ xq, int* __restrict__ topi_g, float* __restrict__ topw_g, sfnx_job* __restrict__ jg,
    sfnx_job* __restrict__ jd, int* __restrict__ njobs_g, float* __restrict__ gu, int8_t* __restrict__ hq_q,
    float* __restrict__ hq_d, int* __restrict__ hq_s, int* __restrict__ route_x, Q8sPlanes sh_gu) {
    constexpr int LPR = lpr_of<TYPE>(), NW = 2 * d2_threads<TYPE>() / WAVE, RPW = WAVE / LPR;
    const int NFB = ff / 32, fb = blockIdx.x % NFB;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    // a dense Q8_0 shared expert's job is job 0 here (the routed jobs follow), so its blocks know their rows before the
    // routing and load them at once: 64 rows of 34 B a block of 32 values against 18 B (Q4_K), it is the longest job
    constexpr bool sh_first = SHQ;
    const bool q8s = SHQ && (int) blockIdx.x < NFB;
    // (held in registers up to 2048 columns; wider rows stream at the dot, as the registers would spill)
    constexpr bool SHR = SHQ && G <= 4;
    Q8sRow<LPR, SHR ? G : 1> ws;
    if constexpr (SHR) {
        const int up_half = threadIdx.x / WAVE >= NW / 2;
        const int srow = (up_half ? ff : 0) + fb * 32 + (up_half ? wave - NW / 2 : wave) * RPW + lane / LPR;
        if (q8s) ws.issue(sh_gu, srow, H, lane % LPR);
    }
    __shared__ float gbuf[32], ubuf[32];
    __shared__ uint32_t junk[WAVE];
    extern __shared__ __align__(16) unsigned char lds[];
    // the logits and the activations requested together
    float lv[NV];
    topk_load<NV>(logits, E / WAVE, lane, lv);
    const Acts a = acts_in(lds, 1, H);
    stage_q8_1(a, xq, nullptr, 1);
    // the next layer's router rows into this XCD's L2 for that layer's K1, while HBM idles through the top-k
    warm_router_rows<2 * d2_threads<TYPE>()>(Wn, E + 1, H, junk);
    int pick;
    uint32_t pord;
    topk_picks<NV>(lv, K, lane, pick, pord);
    const int nr = __popcll(__ballot(lane < K && pick >= 0));
    const int nj = nr + (shared ? 1 : 0);
    // job of this block: routed pick j = jb, the shared job at jb = nr (or first, when dense: then jb = myjob - 1)
    const int myjob = blockIdx.x / NFB, jb = sh_first ? (q8s ? nr : myjob - 1) : myjob;
    const bool has_job = sh_first ? q8s || jb < nr : jb < nj;
    if (!has_job && blockIdx.x >= XCDS) {
        warm_wait();
        return;
    }
    const int ex = jb < nr ? __builtin_amdgcn_readlane(pick, jb) : E, out = jb < nr ? jb : K;
    // the first half of the waves take the 32 gate rows, the second half the matching up rows
    const bool up = wave >= NW / 2;
    const int rw = lane / LPR, ln = lane % LPR, fl = (up ? wave - NW / 2 : wave) * RPW + rw, row = (up ? ff : 0) + fb * 32 + fl;
    const uint8_t* mat = expert_at(A, sa, ex);
    typename RowOf<TYPE, G>::R wr;
    if (has_job && !q8s) RowOf<TYPE, G>::issue(wr, mat, 2 * ff, row, H, ln);
    if (blockIdx.x < XCDS && wave == 0) {   // the routing, published for K3 and the caller, while the rows load
        const float w = topk_weight(pick, pord, K);
        // a copy for K3's workgroups of this XCD (workgroup b on XCD b % 8), read from this XCD's L2
        if (lane < K) {
            route_x[blockIdx.x * 2 * MAX_K + lane] = pick;
            route_x[blockIdx.x * 2 * MAX_K + MAX_K + lane] = __float_as_int(w);
        }
    }
    if (blockIdx.x == 0 && wave == 0) {
        const float w = topk_weight(pick, pord, K);
        if (lane < K) {
            topi_g[lane] = pick;
            topw_g[lane] = w;
        }
        if (lane < nj) {
            const int e = lane < nr ? pick : E, o = lane < nr ? lane : K;
            jg[lane].w = jd[lane].w = e;
            jg[lane].n = jd[lane].n = 1;
            jg[lane].y[0] = 0;
            jg[lane].out[0] = jd[lane].y[0] = jd[lane].out[0] = o;
        }
        if (lane == 0) {
            njobs_g[0] = nj;
            njobs_g[1] = 0;
        }
    }
    if (!has_job) {
        warm_wait();
        return;
    }
    // the staged activations; no memory fence, so each row's groups are dotted as they arrive (the compiler waits for
    // each one) instead of after all of them
    lds_barrier();
    float v;
    if constexpr (SHR) v = group_sum<LPR>(q8s ? ws.dot(a, 0, ln) : wr.dot1(a, ln));
    else if constexpr (SHQ) v = group_sum<LPR>(q8s ? q8s_dot<LPR>(sh_gu, row, H, ln, a, 0) : wr.dot1(a, ln));
    else v = group_sum<LPR>(wr.dot1(a, ln));   // each group as it arrives
    if (ln == 0) {
        gu[(size_t) out * 2 * ff + row] = v;
        (up ? ubuf : gbuf)[fl] = v;
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        const int l = threadIdx.x;
        const float v = silu_f(gbuf[l]) * ubuf[l];
        const float amax = group_max<32>(fabsf(v));
        const float d = amax / 127.0f;
        const int q = amax == 0.0f ? 0 : (int) roundf(v / d);
        const int qs = group_isum<32>(q);
        hq_q[(size_t) out * ff + 32 * fb + l] = (int8_t) q;
        if (l == 0) {
            hq_d[(size_t) out * NFB + fb] = h2f(f2h(d));
            hq_s[(size_t) out * NFB + fb] = qs;
        }
    }
    warm_wait();
}

// ------------------------------------------------------------------------------------------------ K3
// (windows: 512 threads, twice the lane groups of the batch-1 kernel, so a group takes half the tasks)
template <int TYPE, int G2, int NB, int NT>
__global__ void __launch_bounds__(NT) k_dec_down(const uint8_t* __restrict__ A, size_t sa, int T, int H, int E, int K,
                                                        int ff, int shared, const float* __restrict__ logits,
                                                        const int* __restrict__ topi, const float* __restrict__ topw,
                                                        const sfnx_job* __restrict__ jd, const int* __restrict__ njobs,
                                                        const int8_t* __restrict__ hq_q, const float* __restrict__ hq_d,
                                                        const int* __restrict__ hq_s, float* __restrict__ y,
                                                        float* __restrict__ x, int hq_in_lds, Q8sPlanes sh_dn) {
    constexpr int LPR = lpr_of<TYPE>(), GROUPS = NT / LPR;
    const int row0 = blockIdx.x * D3_ROWS, nj = njobs[0], P = T * K, NP = P + T, nbh = ff / 32;
    __shared__ int jw[MAX_P + 1], jn[MAX_P + 1], jout[MAX_P + 1][SFNX_MAXT];
    __shared__ float part[MAX_P + SFNX_MAXT][D3_ROWS];
    __shared__ int ti[MAX_P];
    __shared__ float tw[MAX_P], sg[SFNX_MAXT];
    extern __shared__ __align__(16) unsigned char lds[];   // every pair's h, when the launch gave room for it
    for (int i = threadIdx.x; i < nj; i += NT) {
        jw[i] = jd[i].w;
        jn[i] = jd[i].n;
        for (int s = 0; s < jd[i].n; ++s) jout[i][s] = jd[i].out[s];
    }
    for (int i = threadIdx.x; i < P; i += NT) {
        ti[i] = topi[i];
        tw[i] = topw[i];
    }
    __shared__ float xr[SFNX_MAXT][D3_ROWS];   // the residual rows this block adds to, read with everything else
    for (int i = threadIdx.x; i < T * D3_ROWS; i += NT) xr[i / D3_ROWS][i % D3_ROWS] = x[(size_t) (i / D3_ROWS) * H + row0 + i % D3_ROWS];
    if (shared)
        for (int t = threadIdx.x; t < T; t += NT) sg[t] = sigm_f(logits[(size_t) t * (E + 1) + E]);
    Acts a;
    const bool staged = hq_in_lds != 0;
    if (staged) {
        // every pair's h into LDS by asynchronous global -> LDS copies, all issued before one wait (a copy loop through
        // registers would wait for each of its ~11 rounds in turn): wavefront w copies chunks of 64 lanes, 16 bytes
        // (values) or 4 bytes (scales, sums) a lane
        a = acts_in(lds, NP, ff);
        const int wv = threadIdx.x / WAVE, ln64 = threadIdx.x % WAVE;
        constexpr int NWV = NT / WAVE;
        for (int c = wv; c * WAVE < NP * ff / 16; c += NWV)
            if (c * WAVE + ln64 < NP * ff / 16)
                __builtin_amdgcn_global_load_lds(hq_q + 16 * ((size_t) c * WAVE + ln64),
                                                 (__attribute__((address_space(3))) void*) (a.q + 16 * (size_t) c * WAVE), 16, 0, 0);
        for (int c = wv; c * WAVE < NP * nbh; c += NWV)
            if (c * WAVE + ln64 < NP * nbh) {
                __builtin_amdgcn_global_load_lds(hq_d + c * WAVE + ln64, (__attribute__((address_space(3))) void*) (a.d + c * WAVE), 4, 0, 0);
                __builtin_amdgcn_global_load_lds(hq_s + c * WAVE + ln64, (__attribute__((address_space(3))) void*) (a.s + c * WAVE), 4, 0, 0);
            }
        __builtin_amdgcn_s_waitcnt(0);   // the copies landed (vmcnt), before the barrier below
    }
    __syncthreads();
    const int g = threadIdx.x / LPR, ln = threadIdx.x % LPR;
    // with its own dense Q8_0 matrix the shared expert's job (the last) runs apart, in the reference's q8s sums
    const int nq = sh_dn.q != nullptr && shared ? nj - 1 : nj, ntask = nq * D3_ROWS;
    // the dots, inlined once for h in LDS and once for h in global memory: a pointer that may be either is generic,
    // and every load through it a flat load
    auto dots = [&](const Acts& a) __attribute__((always_inline)) {
    if (nq < nj) {
        const Q8sPlanes Ps = sh_dn;
        for (int task = g; task < T * D3_ROWS; task += GROUPS) {
            const int t = task / D3_ROWS, r = task % D3_ROWS;
            const float v = group_sum<LPR>(q8s_dot<LPR>(Ps, row0 + r, ff, ln, a, P + t));
            if (ln == 0) part[P + t][r] = v;
        }
    }
    for (int t0 = g; t0 < ntask; t0 += GROUPS * NB) {
        typename RowOf<TYPE, G2>::R w[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int task = t0 + b * GROUPS;
            if (task < ntask) {
                const int j = task / D3_ROWS, r = task % D3_ROWS;
                RowOf<TYPE, G2>::load(w[b], expert_at(A, sa, jw[j]), H, row0 + r, ff, ln);
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int task = t0 + b * GROUPS;
            if (task < ntask) {
                const int j = task / D3_ROWS, r = task % D3_ROWS;
                for (int s = 0; s < jn[j]; ++s) {
                    const int pp = jout[j][s];
                    const float v = group_sum<LPR>(w[b].dot(a, pp, ln));
                    if (ln == 0) part[pp][r] = v;
                }
            }
        }
    }
    };
    if (staged) dots(a);
    else dots(Acts{const_cast<int8_t*>(hq_q), const_cast<float*>(hq_d), const_cast<int*>(hq_s), ff});
    __syncthreads();
    for (int i = threadIdx.x; i < T * D3_ROWS; i += NT) {
        const int t = i / D3_ROWS, r = i % D3_ROWS, row = row0 + r;
        float pw[MAX_K], pv[MAX_K];
#pragma unroll
        for (int k = 0; k < MAX_K; ++k) {   // every operand read first, then the chain
            const bool use = k < K && ti[t * K + k] >= 0;
            pw[k] = use ? tw[t * K + k] : 0.f;
            pv[k] = use ? part[t * K + k][r] : 0.f;
        }
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < MAX_K; ++k)
            if (k < K && ti[t * K + k] >= 0) s = fmaf(pw[k], pv[k], s);
        if (shared) s = fmaf(sg[t], part[P + t][r], s);
        y[(size_t) t * H + row] = s;
        x[(size_t) t * H + row] = xr[t][r] + s;
    }
}

// K3 for a window of one row: pair k is pick k, so a task's expert comes straight from the picks (job j = pick j, the
// shared expert's job last).  Every request of the block is issued up front, with one wait: h straight into LDS by
// untracked asynchronous copies (first, so no register holds it and no later wait depends on where the compiler puts
// its loads), the picks, the shared gate's logit, the residual rows, then the weight rows of the picks.
template <int TYPE, int G2, int NB, bool SHQ, int NT3>
__global__ void __launch_bounds__(NT3) k_dec_down1(const uint8_t* __restrict__ A, size_t sa, int H, int E, int K,
                                                         int ff, int shared, const float* __restrict__ logits,
                                                         const int* __restrict__ topi, const float* __restrict__ topw,
                                                         const int8_t* __restrict__ hq_q, const float* __restrict__ hq_d,
                                                         const int* __restrict__ hq_s, float* __restrict__ y,
                                                         float* __restrict__ x, const int* __restrict__ route_x,
                                                         Q8sPlanes sh_dn) {
    constexpr int LPR = lpr_of<TYPE>(), GROUPS = NT3 / LPR;
    const int row0 = blockIdx.x * D3_ROWS, nbh = ff / 32, lane = threadIdx.x % WAVE, tid = threadIdx.x;
    const int g = tid / LPR, ln = tid % LPR;
    __shared__ float part[MAX_K + 1][D3_ROWS];
    extern __shared__ __align__(16) unsigned char lds[];
    const int NP = K + 1, nq = NP * ff / 16, ns = NP * nbh;
    // every pair's h into LDS: 16 bytes of quants a lane, then the (scale, sum) words, wavefront w moving chunks
    // w, w + NT3 / 64, ... of 64 lanes
    const Acts a = acts_in(lds, NP, ff);
    for (int c = tid / WAVE; c * WAVE < nq; c += NT3 / WAVE)
        if (c * WAVE + lane < nq) lds_copy_async<16>(hq_q + 16 * ((size_t) c * WAVE + lane), a.q + 16 * (size_t) c * WAVE);
    for (int c = tid / WAVE; c * WAVE < ns; c += NT3 / WAVE)
        if (c * WAVE + lane < ns) {
            lds_copy_async<4>(hq_d + c * WAVE + lane, a.d + c * WAVE);
            lds_copy_async<4>(hq_s + c * WAVE + lane, a.s + c * WAVE);
        }
    // the picks from the copy K2 left for this XCD
    const int* rx = route_x + (blockIdx.x % XCDS) * 2 * MAX_K;
    const int tp = lane < K ? rx[lane] : -1;
    const float twv = lane < K ? __int_as_float(rx[MAX_K + lane]) : 0.f;
    const float gl = shared ? logits[E] : 0.f;
    const float xr = tid < D3_ROWS ? x[row0 + tid] : 0.f;
    // the picks, then this group's weight rows: task (j, r) = job j's row row0 + r
    const int nr = __popcll(__ballot(lane < K && tp >= 0)), nj = nr + (shared ? 1 : 0), ntask = nj * D3_ROWS;
    typename RowOf<TYPE, G2>::R w[NB];
    int pp[NB], ex[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int j = (g + b * GROUPS) / D3_ROWS;
        ex[b] = __shfl(tp, j < nr ? j : 0);
        pp[b] = j < nr ? j : K;
    }
    // a dense shared expert's task (at most one a lane group: its 8 tasks are consecutive) from its own rows.  Every
    // task's matrix first (with a pointer table, every entry requested before one wait for all)
    global_u8_ptr mats[NB];
    int exb[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) exb[b] = pp[b] < K ? ex[b] : E;
    experts_at<NB>(A, sa, exb, mats);
    Q8sRow<LPR, SHQ ? G2 : 1> wsh;
    int bsh = -1;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int task = g + b * GROUPS, r = task % D3_ROWS;
        if (SHQ && task < ntask && pp[b] == K) {
            wsh.issue(sh_dn, row0 + r, ff, ln);
            bsh = b;
        } else if (task < ntask) {
            RowOf<TYPE, G2>::issue(w[b], (const uint8_t*) mats[b], H, row0 + r, ff, ln);
        }
    }
    // The matrices' addresses escape into an empty statement that may write memory, so no weight load moves below it
    // (the compiler may otherwise sink a load to its use, past the wait, and issue it only then); the one wait (h and
    // every request above), then the barrier for the other wavefronts' copies of h
#pragma unroll
    for (int b = 0; b < NB; ++b) asm volatile("" ::"v"(mats[b]) : "memory");
    if constexpr (SHQ) asm volatile("" ::"v"((global_u8_ptr) sh_dn.q), "v"((const void*) sh_dn.d) : "memory");
    vm_wait<0>();
    lds_barrier();
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int task = g + b * GROUPS;
        if (task < ntask && !(sh_dn.q != nullptr && pp[b] == K)) {
            w[b].prepare(ln);
            const float v = group_sum<LPR>(w[b].dot(a, pp[b], ln));
            if (ln == 0) part[pp[b]][task % D3_ROWS] = v;
        }
    }
    if constexpr (SHQ) {
        if (bsh >= 0) {   // the shared expert's task from its own dense Q8_0 rows (q8s sums)
            const float v = group_sum<LPR>(wsh.dot(a, K, ln));
            if (ln == 0) part[K][(g + bsh * GROUPS) % D3_ROWS] = v;
        }
    }
    // windows with more tasks than one batch (K > 11): the rest, a batch at a time
    for (int t0 = g + NB * GROUPS; t0 < ntask; t0 += GROUPS) {
        const int j = t0 / D3_ROWS, r = t0 % D3_ROWS, e = __shfl(tp, j < nr ? j : 0), q = j < nr ? j : K;
        float v;
        if (sh_dn.q != nullptr && j >= nr) {
            v = group_sum<LPR>(q8s_dot<LPR>(sh_dn, row0 + r, ff, ln, a, K));
        } else {
            typename RowOf<TYPE, G2>::R w1;
            RowOf<TYPE, G2>::load(w1, expert_at(A, sa, j < nr ? e : E), H, row0 + r, ff, ln);
            v = group_sum<LPR>(w1.dot(a, q, ln));
        }
        if (ln == 0) part[q][r] = v;
    }
    __syncthreads();
    // the weighted sum in the reference's fmaf order, then the residual
    if (tid < WAVE) {
        const int r = tid % D3_ROWS;
        float s = 0.f;
        for (int k = 0; k < K; ++k) {
            const int pk = __builtin_amdgcn_readlane(tp, k);
            const float wk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(twv), k));
            if (pk >= 0) s = fmaf(wk, part[k][r], s);
        }
        if (shared) s = fmaf(sigm_f(gl), part[K][r], s);
        if (tid < D3_ROWS) {
            y[row0 + r] = s;
            x[row0 + r] = xr + s;
        }
    }
}

// ------------------------------------------------------------------------------------------------ launch
struct DecArgs {
    uint32_t gu_type, dn_type;
    int H, E, K, ff, shared, T, norm;
    float eps;
    int phases;
    const float* Wn;   // the next layer's router (warmed into L2 for that layer's K1), or null
    Q8sPlanes sh_gu{};   // this layer's shared expert as its own dense Q8_0 matrices, or null planes
    Q8sPlanes sh_dn{};
};

// Optional kernel clock: when on, each decode kernel is launched with a start/stop event pair that the runtime
// stamps at that dispatch's own begin and end, so the elapsed time is the kernel's duration (no launch gaps).
struct KernelClock {
    bool on = false;
    hipEvent_t a[3]{}, b[3]{};
};
KernelClock g_clock;

template <typename F, typename... A>
void launch(int idx, F kern, dim3 grid, dim3 block, size_t shmem, hipStream_t s, A... args) {
    if (g_clock.on)
        hipExtLaunchKernelGGL(kern, grid, block, (uint32_t) shmem, s, g_clock.a[idx], g_clock.b[idx], 0, args...);
    else
        hipLaunchKernelGGL(kern, grid, block, shmem, s, args...);
}

template <int NC, int TT>
void launch_k1(const DecArgs& d, const sfnx_moe_layer_w& w, float* x, const DecLayout& L, char* ws, hipStream_t s) {
    const int rows = d.E + 1;
    launch(0, k_dec_router<NC, TT>, dim3((rows + D1_WAVES - 1) / D1_WAVES), dim3(D1_THREADS * d1_groups<TT>()), 0, s,
        w.W, x, d.T, d.E, d.eps, d.norm, (float*) (ws + L.logits), (uint8_t*) (ws + L.xq));
}
template <int TYPE, int G> void launch_k2_tt1(const DecArgs&, const sfnx_moe_layer_w&, const DecLayout&, char*, hipStream_t);
template <int TYPE, int G, int TT>
void launch_k2(const DecArgs& d, const sfnx_moe_layer_w& w, const DecLayout& L, char* ws, hipStream_t s) {
    if constexpr (TT == 1) {
        launch_k2_tt1<TYPE, G>(d, w, L, ws, s);
    } else {
        const int njmax = d.T * d.K + (d.shared ? 1 : 0);
        // the routing once (K1b), then the experts
        hipLaunchKernelGGL(k_dec_route, dim3(1), dim3(DR_THREADS), 0, s, d.T, d.E, d.K, d.shared,
            (const float*) (ws + L.logits), (int*) (ws + L.topi), (float*) (ws + L.topw), (sfnx_job*) (ws + L.jg),
            (sfnx_job*) (ws + L.jd), (int*) (ws + L.njobs));
        launch(1, k_dec_experts<TYPE, G, TT>, dim3(njmax * (d.ff / 32)), dim3(2 * d2_threads<TYPE>()), acts_bytes(TT, d.H), s,
            (const uint8_t*) w.gu, w.gu_stride, d.H, d.E, d.ff, (const uint8_t*) (ws + L.xq), (const sfnx_job*) (ws + L.jg),
            (const int*) (ws + L.njobs), (float*) (ws + L.gu), (int8_t*) (ws + L.hq_q), (float*) (ws + L.hq_d),
            (int*) (ws + L.hq_s), d.sh_gu);
    }
}
template <int TYPE, int G, int NV, bool SHQ>
void launch_k2_one(const DecArgs& d, const sfnx_moe_layer_w& w, const DecLayout& L, char* ws, hipStream_t s) {
    const int njmax = d.K + (d.shared ? 1 : 0);
    launch(1, k_dec_experts1<TYPE, G, NV, SHQ>, dim3(njmax * (d.ff / 32)), dim3(2 * d2_threads<TYPE>()), acts_bytes(1, d.H), s,
        (const uint8_t*) w.gu, w.gu_stride, d.Wn, d.H, d.E, d.K, d.ff, d.shared, (const float*) (ws + L.logits),
        (const uint8_t*) (ws + L.xq), (int*) (ws + L.topi), (float*) (ws + L.topw), (sfnx_job*) (ws + L.jg),
        (sfnx_job*) (ws + L.jd), (int*) (ws + L.njobs), (float*) (ws + L.gu), (int8_t*) (ws + L.hq_q),
        (float*) (ws + L.hq_d), (int*) (ws + L.hq_s), (int*) (ws + L.route_x), d.sh_gu);
}
template <int TYPE, int G>
void launch_k2_tt1(const DecArgs& d, const sfnx_moe_layer_w& w, const DecLayout& L, char* ws, hipStream_t s) {
    if (d.sh_gu.q) {
        if (d.E <= 256) launch_k2_one<TYPE, G, 4, true>(d, w, L, ws, s);
        else if (d.E <= 512) launch_k2_one<TYPE, G, 8, true>(d, w, L, ws, s);
        else launch_k2_one<TYPE, G, 16, true>(d, w, L, ws, s);
    } else {
        if (d.E <= 256) launch_k2_one<TYPE, G, 4, false>(d, w, L, ws, s);
        else if (d.E <= 512) launch_k2_one<TYPE, G, 8, false>(d, w, L, ws, s);
        else launch_k2_one<TYPE, G, 16, false>(d, w, L, ws, s);
    }
}
template <int TYPE, int G2>
void launch_k3_one(const DecArgs& d, const sfnx_moe_layer_w& w, float* x, const DecLayout& L, char* ws, hipStream_t s) {
    // 512 threads: 64 lane groups (K-quants) or 32, so 11 jobs x 8 rows are one batch of 2 or 3 tasks a group
    constexpr int NT3 = 512, NB = is_kquant(TYPE) ? 2 : 3;
    auto kern = d.sh_dn.q ? k_dec_down1<TYPE, G2, NB, true, NT3> : k_dec_down1<TYPE, G2, NB, false, NT3>;
    launch(2, kern, dim3(d.H / D3_ROWS), dim3(NT3), acts_bytes(d.K + 1, d.ff), s,
        (const uint8_t*) w.dn, w.dn_stride, d.H, d.E, d.K, d.ff, d.shared, (const float*) (ws + L.logits),
        (const int*) (ws + L.topi), (const float*) (ws + L.topw), (const int8_t*) (ws + L.hq_q),
        (const float*) (ws + L.hq_d), (const int*) (ws + L.hq_s), (float*) (ws + L.y), x, (const int*) (ws + L.route_x),
        d.sh_dn);
}
template <int TYPE, int G2, int NB>
void launch_k3(const DecArgs& d, const sfnx_moe_layer_w& w, float* x, const DecLayout& L, char* ws, hipStream_t s) {
    if (d.T == 1) {
        launch_k3_one<TYPE, G2>(d, w, x, L, ws, s);
        return;
    }
    const int NP = d.T * d.K + d.T;
    const size_t hq_lds = acts_bytes(NP, d.ff);
    // every pair's h in LDS when it fits beside the kernel's own ~30 KB (160 KB a workgroup on gfx950; past 64 KB the
    // kernel must be allowed the larger dynamic size first), else read from L2 per task
    constexpr size_t HQ_LDS_MAX = 120 * 1024;
    // 1024 threads (4 wavefronts a SIMD: the per-pair dot chains are latency-bound) where 128 registers hold a lane's
    // tasks (FF 512; not Q5_K, whose rows carry their fifth bits)
    constexpr int NT = G2 == 1 && TYPE != SFNX_Q5_K ? 1024 : 512;
    static bool big_lds = hipFuncSetAttribute((const void*) k_dec_down<TYPE, G2, NB, NT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                              (int) HQ_LDS_MAX) == hipSuccess;
    const bool staged = hq_lds <= (big_lds ? HQ_LDS_MAX : 32 * 1024);
    launch(2, k_dec_down<TYPE, G2, NB, NT>, dim3(d.H / D3_ROWS), dim3(NT), staged ? hq_lds : 0, s,
        (const uint8_t*) w.dn, w.dn_stride, d.T, d.H, d.E, d.K, d.ff, d.shared, (const float*) (ws + L.logits),
        (const int*) (ws + L.topi), (const float*) (ws + L.topw), (const sfnx_job*) (ws + L.jd), (const int*) (ws + L.njobs),
        (const int8_t*) (ws + L.hq_q), (const float*) (ws + L.hq_d), (const int*) (ws + L.hq_s), (float*) (ws + L.y), x,
        staged ? 1 : 0, d.sh_dn);
}

template <int TT>
void launch_layer_tt(const DecArgs& d, const sfnx_moe_layer_w& w, float* x, const DecLayout& L, char* ws, hipStream_t s) {
    if (d.phases & 1) switch (d.H) {
        case 1024: launch_k1<4, TT>(d, w, x, L, ws, s); break;
        case 2048: launch_k1<8, TT>(d, w, x, L, ws, s); break;
        case 2560: launch_k1<10, TT>(d, w, x, L, ws, s); break;
        case 4096: launch_k1<16, TT>(d, w, x, L, ws, s); break;
        default: throw std::runtime_error("hidden size must be 1024, 2048, 2560 or 4096");
    }
    const int G = d.H / 512;
#define SFNX_K2(TY)                                                       \
    switch (G) {                                                          \
        case 2: launch_k2<TY, 2, TT>(d, w, L, ws, s); break;              \
        case 4: launch_k2<TY, 4, TT>(d, w, L, ws, s); break;              \
        case 5: launch_k2<TY, 5, TT>(d, w, L, ws, s); break;              \
        case 8: launch_k2<TY, 8, TT>(d, w, L, ws, s); break;              \
        default: throw std::runtime_error("hidden size must be 1024, 2048, 2560 or 4096"); \
    }
    if (d.phases & 2) {
        switch (d.gu_type) {
            case SFNX_Q4_K: SFNX_K2(SFNX_Q4_K) break;
            case SFNX_Q5_K: SFNX_K2(SFNX_Q5_K) break;
            case SFNX_Q4_0: SFNX_K2(SFNX_Q4_0) break;
            case SFNX_Q5_1: SFNX_K2(SFNX_Q5_1) break;
            default: SFNX_K2(SFNX_Q8_0) break;
        }
    }
#undef SFNX_K2
    // down tasks a lane group loads together: every job's 8 rows in one batch at T = 1
    constexpr int NB = TT == 1 ? 3 : 4, NB2 = NB;
    if (!(d.phases & 4)) return;
    if (d.dn_type == SFNX_Q4_K) {
        if (d.ff == 512) launch_k3<SFNX_Q4_K, 1, NB>(d, w, x, L, ws, s);
        else launch_k3<SFNX_Q4_K, 2, NB2>(d, w, x, L, ws, s);
    } else if (d.dn_type == SFNX_Q5_K) {
        if (d.ff == 512) launch_k3<SFNX_Q5_K, 1, NB>(d, w, x, L, ws, s);
        else launch_k3<SFNX_Q5_K, 2, NB2>(d, w, x, L, ws, s);
    } else if (d.dn_type == SFNX_Q4_0) {
        if (d.ff == 512) launch_k3<SFNX_Q4_0, 1, NB>(d, w, x, L, ws, s);
        else launch_k3<SFNX_Q4_0, 2, NB2>(d, w, x, L, ws, s);
    } else if (d.dn_type == SFNX_Q5_1) {
        if (d.ff == 512) launch_k3<SFNX_Q5_1, 1, NB>(d, w, x, L, ws, s);
        else launch_k3<SFNX_Q5_1, 2, NB2>(d, w, x, L, ws, s);
    } else {
        if (d.ff == 512) launch_k3<SFNX_Q8_0, 1, NB>(d, w, x, L, ws, s);
        else launch_k3<SFNX_Q8_0, 2, NB2>(d, w, x, L, ws, s);
    }
}

}  // namespace
}  // namespace sfnx

using namespace sfnx;


extern "C" int sfnx_kernel_clock(int enable) {
    return guarded("sfnx_kernel_clock", [&] {
        if (enable && !g_clock.a[0])
            for (int i = 0; i < 3; ++i) {
                check(hipEventCreate(&g_clock.a[i]), "hipEventCreate");
                check(hipEventCreate(&g_clock.b[i]), "hipEventCreate");
            }
        g_clock.on = enable != 0;
    });
}

extern "C" int sfnx_kernel_clock_read(float* us) {
    return guarded("sfnx_kernel_clock_read", [&] {
        require(g_clock.a[0] != nullptr && us != nullptr, "kernel clock never enabled");
        for (int i = 0; i < 3; ++i) {
            check(hipEventSynchronize(g_clock.b[i]), "hipEventSynchronize");
            float ms = 0.f;
            check(hipEventElapsedTime(&ms, g_clock.a[i], g_clock.b[i]), "hipEventElapsedTime");
            us[i] = ms * 1000.f;
        }
    });
}

extern "C" size_t sfnx_moe_decode_workspace(int T, int H, int E, int K, int ff, size_t* offsets) {
    if (T < 1 || T > SFNX_MAXT) return 0;
    const DecLayout L = dec_layout(H, E, K, ff);
    if (offsets) {
        const size_t o[13] = {L.logits, L.xq, L.topi, L.topw, L.jg, L.jd, L.njobs, L.gu, L.hq_q, L.hq_d, L.hq_s, L.y, L.total};
        for (int i = 0; i < 13; ++i) offsets[i] = o[i];
    }
    return L.total;
}

namespace {
void moe_decode(const sfnx_moe_layer_w* layers, const sfnx_moe_shared_q8s* sh, int n_layers, uint32_t gu_type,
                uint32_t dn_type, int H, int E, int K, int ff, int shared, float* x, int T, int norm, float eps, void* ws,
                size_t ws_bytes, int phases, void* st) {
    {
        const uint32_t type = gu_type;
        require(expert_type_ok(gu_type) && expert_type_ok(dn_type), TYPE_MSG);
        require(T >= 1 && T <= SFNX_MAXT, "T out of range (1..16)");
        require(E >= WAVE && E % WAVE == 0 && E <= MAX_E, "E must be a multiple of 64, at most 1024");
        require(K >= 1 && K <= MAX_K && K <= E, "K out of range (1..16)");
        require(H == 1024 || H == 2048 || H == 2560 || H == 4096, "hidden size must be 1024, 2048, 2560 or 4096");
        require(ff == 512 || ff == 1024, "FF must be 512 or 1024");
        require(T * K <= (is_kquant(type) ? 256 : 512), "T K picks exceed the block");
        const DecLayout L = dec_layout(H, E, K, ff);
        require(ws != nullptr && ws_bytes >= L.total, "workspace smaller than sfnx_moe_decode_workspace()");
        require(n_layers >= 0 && (n_layers == 0 || layers != nullptr), "no layers");
        for (int l = 0; l < n_layers; ++l) {
            require(layers[l].W && layers[l].gu && layers[l].dn, "a layer's weights are missing");
            require(stride_ok(layers[l].gu_stride, row_bytes(type, H) * 2 * (size_t) ff), "gate|up stride smaller than a matrix");
            require(stride_ok(layers[l].dn_stride, row_bytes(dn_type, ff) * (size_t) H), "down stride smaller than a matrix");
            if (sh) require(sh[l].gu.q && sh[l].gu.d && sh[l].dn.q && sh[l].dn.d, "a layer's shared expert matrices are missing");
        }
        const DecArgs d{gu_type, dn_type, H, E, K, ff, shared ? 1 : 0, T, norm ? 1 : 0, eps, phases ? phases : 7, nullptr};
        hipStream_t s = stream_of(st);
        char* w = (char*) ws;
        for (int l = 0; l < n_layers; ++l) {
            DecArgs dl = d;
            dl.Wn = l + 1 < n_layers ? layers[l + 1].W : nullptr;
            if (sh) {
                dl.sh_gu = Q8sPlanes{sh[l].gu.q, sh[l].gu.d};
                dl.sh_dn = Q8sPlanes{sh[l].dn.q, sh[l].dn.d};
            }
            if (T == 1) launch_layer_tt<1>(dl, layers[l], x, L, w, s);
            else if (T <= 4) launch_layer_tt<4>(dl, layers[l], x, L, w, s);
            else launch_layer_tt<16>(dl, layers[l], x, L, w, s);
        }
    }
}
}  // namespace

extern "C" int sfnx_moe_decode2(const sfnx_moe_layer_w* layers, int n_layers, uint32_t gu_type, uint32_t dn_type, int H,
                                int E, int K, int ff, int shared, float* x, int T, int norm, float eps, void* ws,
                                size_t ws_bytes, int phases, void* st) {
    return guarded("sfnx_moe_decode", [&] {
        moe_decode(layers, nullptr, n_layers, gu_type, dn_type, H, E, K, ff, shared, x, T, norm, eps, ws, ws_bytes, phases, st);
    });
}

extern "C" int sfnx_moe_decode_q8s(const sfnx_moe_layer_w* layers, const sfnx_moe_shared_q8s* shared_w, int n_layers,
                                   uint32_t gu_type, uint32_t dn_type, int H, int E, int K, int ff, float* x, int T,
                                   int norm, float eps, void* ws, size_t ws_bytes, int phases, void* st) {
    return guarded("sfnx_moe_decode_q8s", [&] {
        require(shared_w != nullptr || n_layers == 0, "no shared expert matrices");
        moe_decode(layers, shared_w, n_layers, gu_type, dn_type, H, E, K, ff, 1, x, T, norm, eps, ws, ws_bytes, phases, st);
    });
}

extern "C" int sfnx_moe_decode(const sfnx_moe_layer_w* layers, int n_layers, uint32_t type, int H, int E, int K, int ff,
                               int shared, float* x, int T, int norm, float eps, void* ws, size_t ws_bytes, int phases,
                               void* st) {
    return sfnx_moe_decode2(layers, n_layers, type, type, H, E, K, ff, shared, x, T, norm, eps, ws, ws_bytes, phases, st);
}

// ------------------------------------------------------------------------------------------------ no allocation
// The decode workspace as a file-scope device array, for callers that cannot allocate.  Its host-side name is no
// device address: host code uses only the address hipGetSymbolAddress returns, fetched once per device.
namespace {
constexpr size_t NOALLOC_BYTES = 4u << 20;
__device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];
constexpr int NOALLOC_DEVS = 64;
void* g_scratch[NOALLOC_DEVS] = {};
// the guard against calls that overlap on one GPU: an event recorded after each (uncaptured) call, and its stream
hipEvent_t g_done[NOALLOC_DEVS] = {};
hipStream_t g_last[NOALLOC_DEVS] = {};
bool g_used[NOALLOC_DEVS] = {};
std::mutex g_scratch_mu;
int device_index() {
    int dev = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < NOALLOC_DEVS, "device index past the library's table");
    return dev;
}
void* scratch_of_device(int dev) {
    if (!g_scratch[dev]) {
        void* p = nullptr;
        check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress (decode scratch)");
        g_scratch[dev] = p;
        check(hipEventCreateWithFlags(&g_done[dev], hipEventDisableTiming), "hipEventCreateWithFlags (decode scratch)");
    }
    return g_scratch[dev];
}
}  // namespace

extern "C" int sfnx_moe_decode_noalloc(const sfnx_moe_layer_w* layers, int n_layers, uint32_t gu_type, uint32_t dn_type,
                                       int H, int E, int K, int ff, int shared, float* x, int T, int norm, float eps,
                                       void* st) {
    return guarded("sfnx_moe_decode_noalloc", [&] {
        const DecLayout L = dec_layout(H, E, K, ff);
        require(L.total <= NOALLOC_BYTES, "shape needs a decode workspace larger than the library's 4 MiB scratch");
        // Every call on a GPU shares the one scratch array.  A call on another stream than the last uncaptured call's
        // is refused while that call still runs (the two would race on the array); calls on one stream are ordered by
        // the stream.  Under graph capture the check is left to the caller (the captured work runs at replay).
        hipStream_t s = stream_of(st);
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        check(hipStreamIsCapturing(s, &cap), "hipStreamIsCapturing");
        const bool captured = cap != hipStreamCaptureStatusNone;
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        const int dev = device_index();
        void* ws = scratch_of_device(dev);
        if (!captured && g_used[dev] && g_last[dev] != s) {
            const hipError_t q = hipEventQuery(g_done[dev]);
            if (q == hipErrorNotReady)
                throw std::runtime_error("a call on another stream still runs on this GPU's scratch array (calls that overlap on one GPU race)");
            if (q != hipSuccess) check(q, "hipEventQuery");
        }
        moe_decode(layers, nullptr, n_layers, gu_type, dn_type, H, E, K, ff, shared, x, T, norm, eps, ws, NOALLOC_BYTES, 0, st);
        if (!captured) {
            check(hipEventRecord(g_done[dev], s), "hipEventRecord");
            g_last[dev] = s;
            g_used[dev] = true;
        }
    });
}
