// Activations and routing: q8_1 quantization, the decode router (logits, top-k, jobs in one launch), the prompt path's
// router logits and permutation, and the weighted combine.
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
// block to finish takes the top-K of every token and builds the jobs (first-pick order, rows in pair order)
template <int NC, int TT>
__global__ void __launch_bounds__(RR_THREADS) k_router_route(const float* __restrict__ W, const float* __restrict__ x,
                                                            float* __restrict__ logits, int T, int E, int K,
                                                            int* __restrict__ topi, float* __restrict__ topw,
                                                            sfnx_job* __restrict__ gu, sfnx_job* __restrict__ dn,
                                                            int* __restrict__ njobs, int shared) {
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
    if (!last) return;
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
    __shared__ unsigned char first[MAX_P];
    __shared__ int jobof[MAX_E];
    PickSlot ps;
    const int nr = pick_slots(ex, P, first, jobof, ps);
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
}

// any number of tokens: a wavefront per row and token block of up to 8 tokens (the prompt path's router)
template <int NC>
__global__ void __launch_bounds__(RR_THREADS) k_router_logits(const float* __restrict__ W, const float* __restrict__ x,
                                                             float* __restrict__ logits, int T, int L) {
    constexpr int H = NC * 4 * WAVE, TB = 8;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int row = blockIdx.x * RR_WAVES + wave, t0 = blockIdx.y * TB;
    if (row >= L) return;
    float4 wv[NC];
    row_load<NC>(W + (size_t) row * H, lane, wv);
    for (int t = t0; t < min(T, t0 + TB); ++t) {
        const float s = row_dot<NC>(wv, x + (size_t) t * H, lane);
        if (lane == 0) logits[(size_t) t * L + row] = s;
    }
}

// ------------------------------------------------------------------------------------------------ prompt routing
// src/prefill.cu:191-221 k_pf_top10: a wavefront per token
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
__global__ void k_fill_int(int* p, int n, int v) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}
// src/prefill.cu:223-226 k_pf_count
__global__ void k_pf_count(const int* __restrict__ topi, int P, int* __restrict__ cnt) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p < P && topi[p] >= 0) atomicAdd(&cnt[topi[p]], 1);
}
// src/prefill.cu:228-242 k_pf_jobbase: one block of E threads (E <= 1024), an inclusive scan of ceil(cnt / 64)
__global__ void k_pf_jobbase(const int* __restrict__ cnt, int* __restrict__ jbase, int* __restrict__ njobs, int E, int C,
                             int shared) {
    __shared__ int s[MAX_E];
    const int e = threadIdx.x;
    const int nj = e < E ? (cnt[e] + SFNX_PF_JOB - 1) / SFNX_PF_JOB : 0;
    s[e] = nj;
    __syncthreads();
    for (int o = 1; o < (int) blockDim.x; o <<= 1) {
        const int a = e >= o ? s[e - o] : 0;
        __syncthreads();
        s[e] += a;
        __syncthreads();
    }
    if (e < E) jbase[e] = s[e] - nj;
    if (e == (int) blockDim.x - 1) njobs[0] = s[e] + (shared ? (C + SFNX_PF_JOB - 1) / SFNX_PF_JOB : 0);
}
// src/prefill.cu:248-279 k_pf_fill: a block per expert scans the pairs in index order, a ballot prefix per pass, so a
// pair always lands in the same job and slot
constexpr int PF_FILL_THREADS = 256;
__global__ void __launch_bounds__(PF_FILL_THREADS) k_pf_fill(const int* __restrict__ topi, int P, int K,
                                                            const int* __restrict__ cnt, const int* __restrict__ jbase,
                                                            sfnx_bigjob* __restrict__ gu, sfnx_bigjob* __restrict__ dn) {
    const int e = blockIdx.x, tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int ce = cnt[e];
    if (ce == 0) return;
    __shared__ int wcount[PF_FILL_THREADS / WAVE];
    int base = 0;
    for (int p0 = 0; p0 < P; p0 += PF_FILL_THREADS) {
        const int p = p0 + tid;
        const bool mine = p < P && topi[p] == e;
        const uint64_t m = __ballot(mine);
        if (lane == 0) wcount[wave] = __popcll(m);
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int w = 0; w < PF_FILL_THREADS / WAVE; ++w) {
            before += w < wave ? wcount[w] : 0;
            total += wcount[w];
        }
        if (mine) {
            const int s = base + before + __popcll(m & ((1ull << lane) - 1ull));
            const int j = jbase[e] + s / SFNX_PF_JOB, k = s % SFNX_PF_JOB;
            gu[j].y[k] = p / K;
            gu[j].out[k] = p;
            dn[j].y[k] = p;
            dn[j].out[k] = p;
            if (k == 0) {
                const int n = min(SFNX_PF_JOB, ce - (s / SFNX_PF_JOB) * SFNX_PF_JOB);
                gu[j].w = dn[j].w = e;
                gu[j].n = dn[j].n = n;
            }
        }
        base += total;
        __syncthreads();
    }
}
// the shared expert's jobs after the routed ones: tokens in order, 64 a job
__global__ void k_pf_shared(int C, int P, int E, const int* __restrict__ njobs, sfnx_bigjob* __restrict__ gu,
                            sfnx_bigjob* __restrict__ dn) {
    const int nsh = (C + SFNX_PF_JOB - 1) / SFNX_PF_JOB, j0 = njobs[0] - nsh;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= C) return;
    const int j = j0 + t / SFNX_PF_JOB, k = t % SFNX_PF_JOB;
    gu[j].y[k] = t;
    gu[j].out[k] = dn[j].y[k] = dn[j].out[k] = P + t;
    if (k == 0) {
        gu[j].w = dn[j].w = E;
        gu[j].n = dn[j].n = min(SFNX_PF_JOB, C - t);
    }
}

// ------------------------------------------------------------------------------------------------ combine
// src/kernels.cu:797-803 ring_x / src/prefill.cu:476-484 k_pfr_addend
__global__ void k_combine(const float* __restrict__ part, const float* __restrict__ topw, const int* __restrict__ topi,
                          const float* __restrict__ logits, float* __restrict__ y, int T, int H, int E, int K, int shared) {
    const size_t n = (size_t) T * H;
    for (size_t q = blockIdx.x * (size_t) blockDim.x + threadIdx.x; q < n; q += (size_t) gridDim.x * blockDim.x) {
        const int t = (int) (q / H), i = (int) (q % H);
        float s = 0.f;
        for (int k = 0; k < K; ++k)
            if (topi[t * K + k] >= 0) s = fmaf(topw[t * K + k], part[((size_t) t * K + k) * H + i], s);
        if (shared) s = fmaf(sigm_f(logits[(size_t) t * (E + 1) + E]), part[((size_t) T * K + t) * H + i], s);
        y[q] = s;
    }
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

extern "C" int sfnx_router_logits(const float* W, const float* x, float* logits, int T, int H, int L, void* st) {
    return guarded("sfnx_router_logits", [&] {
        require(H % 256 == 0, "H must be a multiple of 256");
        if (T <= 0 || L <= 0) return;
        const dim3 g((L + RR_WAVES - 1) / RR_WAVES, (T + 7) / 8);
        hipStream_t s = stream_of(st);
        switch (H / 256) {
            case 4: k_router_logits<4><<<g, RR_THREADS, 0, s>>>(W, x, logits, T, L); break;
            case 8: k_router_logits<8><<<g, RR_THREADS, 0, s>>>(W, x, logits, T, L); break;
            case 10: k_router_logits<10><<<g, RR_THREADS, 0, s>>>(W, x, logits, T, L); break;
            case 16: k_router_logits<16><<<g, RR_THREADS, 0, s>>>(W, x, logits, T, L); break;
            default: throw std::runtime_error("hidden size must be 1024, 2048, 2560 or 4096");
        }
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
        k_fill_int<<<(E + 255) / 256, 256, 0, s>>>(cnt, E, 0);
        k_pf_count<<<(P + 255) / 256, 256, 0, s>>>(topi, P, cnt);
        int nt = 64;
        while (nt < E) nt *= 2;
        k_pf_jobbase<<<1, nt, 0, s>>>(cnt, jbase, njobs, E, C, shared);
        k_pf_fill<<<E, PF_FILL_THREADS, 0, s>>>(topi, P, K, cnt, jbase, jobs_gu, jobs_dn);
        if (shared) k_pf_shared<<<(C + 255) / 256, 256, 0, s>>>(C, P, E, njobs, jobs_gu, jobs_dn);
    });
}

extern "C" int sfnx_moe_combine(const float* part, const float* topw, const int* topi, const float* logits, float* y, int T,
                                int H, int E, int K, int shared, void* st) {
    return guarded("sfnx_moe_combine", [&] {
        if (T <= 0) return;
        const size_t n = (size_t) T * H;
        k_combine<<<(unsigned) std::min<size_t>((n + 255) / 256, 8192), 256, 0, stream_of(st)>>>(part, topw, topi, logits, y, T,
                                                                                                 H, E, K, shared);
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
