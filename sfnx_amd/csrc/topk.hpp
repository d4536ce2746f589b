// Routing building blocks: a wavefront's top-K of one token's expert logits, and the decode job numbering.
#pragma once
#include "common.hpp"

namespace sfnx {

constexpr int MAX_E = 1024, MAX_K = 16, MAX_P = SFNX_MAXT * MAX_K;

// Wavefront reductions by DPP row operations (quad swaps, half-row and row mirrors, then the row broadcasts 15 and 31);
// lane 63 holds the result, returned to every lane.  wave_max ignores NaN (v_max_f32's maxNum rule).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __int_as_float(dpp_mov<0xB1>(__float_as_int(v))));          // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, __int_as_float(dpp_mov<0x4E>(__float_as_int(v))));          // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, __int_as_float(dpp_mov<0x141>(__float_as_int(v))));         // row_half_mirror
    v = fmaxf(v, __int_as_float(dpp_mov<0x140>(__float_as_int(v))));         // row_mirror
    v = fmaxf(v, __int_as_float(dpp_mov<0x142, 0xa>(__float_as_int(v))));    // row_bcast:15 into rows 1 and 3
    v = fmaxf(v, __int_as_float(dpp_mov<0x143, 0xc>(__float_as_int(v))));    // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ int wave_min(int v) {
    v = min(v, dpp_mov<0xB1>(v));
    v = min(v, dpp_mov<0x4E>(v));
    v = min(v, dpp_mov<0x141>(v));
    v = min(v, dpp_mov<0x140>(v));
    v = min(v, dpp_mov<0x142, 0xa>(v));
    v = min(v, dpp_mov<0x143, 0xc>(v));
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#define SFNX_KSTAGE(CTRL, ROWS)                                                                              \
    {                                                                                                        \
        const uint32_t hi = (uint32_t) dpp_mov<CTRL, ROWS>((int) (k >> 32)), lo = (uint32_t) dpp_mov<CTRL, ROWS>((int) k); \
        const uint64_t o = ((uint64_t) hi << 32) | lo;                                                       \
        k = o > k ? o : k;                                                                                   \
    }
    SFNX_KSTAGE(0xB1, 0xf)
    SFNX_KSTAGE(0x4E, 0xf)
    SFNX_KSTAGE(0x141, 0xf)
    SFNX_KSTAGE(0x140, 0xf)
    SFNX_KSTAGE(0x142, 0xa)
    SFNX_KSTAGE(0x143, 0xc)
#undef SFNX_KSTAGE
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readlane((int) (k >> 32), 63);
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readlane((int) k, 63);
    return ((uint64_t) hi << 32) | lo;
}

// a logit and its index as one 64-bit key whose unsigned order is the pick order: the float's bits made monotone
// (-0 taken as +0, so equal values compare equal) above the complemented index (the lower index wins a tie); NaN and
// -inf, never taken, become 0
__device__ __forceinline__ uint64_t pick_key(float v, int idx) {
    if (v != v || v == -INFINITY) return 0;
    const uint32_t u = __float_as_uint(v + 0.0f);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t) ord << 32) | (uint32_t) ~idx;
}
__device__ __forceinline__ float key_value(uint64_t k) {
    const uint32_t ord = (uint32_t) (k >> 32);
    return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
}

// unsigned maximum / minimum over the wavefront by DPP row operations, every lane's result in lane 63, returned to all;
// lanes a row mask leaves out read the operation's identity
template <int CTRL, int ROWS = 0xf> __device__ __forceinline__ uint32_t dpp_or(uint32_t v, uint32_t identity) {
    return (uint32_t) __builtin_amdgcn_update_dpp((int) identity, (int) v, CTRL, ROWS, 0xf, false);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_or<0xB1>(v, 0u));
    v = max(v, dpp_or<0x4E>(v, 0u));
    v = max(v, dpp_or<0x141>(v, 0u));
    v = max(v, dpp_or<0x140>(v, 0u));
    v = max(v, dpp_or<0x142, 0xa>(v, 0u));
    v = max(v, dpp_or<0x143, 0xc>(v, 0u));
    return (uint32_t) __builtin_amdgcn_readlane((int) v, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, dpp_or<0xB1>(v, ~0u));
    v = min(v, dpp_or<0x4E>(v, ~0u));
    v = min(v, dpp_or<0x141>(v, ~0u));
    v = min(v, dpp_or<0x140>(v, ~0u));
    v = min(v, dpp_or<0x142, 0xa>(v, ~0u));
    v = min(v, dpp_or<0x143, 0xc>(v, ~0u));
    return (uint32_t) __builtin_amdgcn_readlane((int) v, 63);
}

// one token's E = 64 NV logits into registers, lane l holding experts l + 64 i (i < nv; the rest NaN)
template <int NV, bool AGENT = false>
__device__ __forceinline__ void topk_load(const float* lg, int nv, int lane, float (&lv)[NV]) {
#pragma unroll
    for (int i = 0; i < NV; ++i) lv[i] = i >= nv ? NAN : AGENT ? load_agent(lg + lane + WAVE * i) : lg[lane + WAVE * i];
}

// The top-K of one token's logits (lane l holds experts l + 64 i) by one wavefront: K rounds of the largest untaken
// value, the lowest index among equal values (the reference's strict `>` scan, then `oi < bi` across lanes); NaN and
// -inf are never taken (src/moe.cuh:128-162, src/prefill.cu:191-221).  A round is a DPP maximum over the lanes' heads,
// the winner moving to its next key.  Lane k < K returns pick k; a round with nothing left gives index -1.
//
// The rounds run on one 32-bit key: the value's order bits above bit 10 (its upper 22 bits), the complemented index
// below (E <= 1024), each lane's keys sorted once.  Those rounds pick the top K exactly in that key's order.  The exact
// top K can differ only if an untaken value shares its upper 22 bits with the last pick, or two picks share them (their
// order then rests on the dropped bits): both are checked, and either one redoes the selection on exact 64-bit keys.
template <int NV>
__device__ inline void topk_picks(const float (&lv)[NV], int K, int lane, int& pick, uint32_t& pord) {
    uint32_t tk[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t o = (uint32_t) (pick_key(lv[i], 0) >> 32);
        tk[i] = o ? (o & 0xFFFFFC00u) | (1023u - (uint32_t) (lane + WAVE * i)) : 0u;
    }
    // descending bitonic sort of the lane's keys
#pragma unroll
    for (int k = 2; k <= NV; k *= 2)
#pragma unroll
        for (int j = k / 2; j > 0; j /= 2)
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    const uint32_t a = tk[i], b = tk[l];
                    const bool desc = (i & k) == 0;
                    tk[i] = desc ? max(a, b) : min(a, b);
                    tk[l] = desc ? min(a, b) : max(a, b);
                }
            }
    uint32_t mk = 0;
    for (int k = 0; k < K; ++k) {
        const uint32_t best = wave_max_u32(tk[0]);
        if (lane == k) mk = best;
        // the winner's keys move up a slot: one v_cndmask a slot on the winner mask (written as such: the compiler
        // otherwise turns the shift into per-slot index selects, several times longer)
        const uint64_t won = __ballot(tk[0] == best);
        asm volatile("s_nop 2" ::"s"(won));   // the mask's VALU write before its reads as a select mask
#pragma unroll
        for (int i = 0; i + 1 < NV; ++i) asm volatile("v_cndmask_b32_e64 %0, %0, %1, %2" : "+v"(tk[i]) : "v"(tk[i + 1]), "s"(won));
        asm volatile("v_cndmask_b32_e64 %0, %0, 0, %1" : "+v"(tk[NV - 1]) : "s"(won));
    }
    // each pick's exact order bits, from the lane and slot that held it
    const uint32_t pi = mk ? 1023u - (mk & 1023u) : ~0u;
    uint32_t po = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t o = (uint32_t) __shfl((int) (uint32_t) (pick_key(lv[i], 0) >> 32), (int) (pi & 63u));
        po = (pi >> 6) == (uint32_t) i ? o : po;
    }
    const uint64_t pk = mk ? ((uint64_t) po << 32) | ~pi : 0;
    const uint32_t nlo = (uint32_t) dpp_mov<0x101>((int) (uint32_t) pk), nhi = (uint32_t) dpp_mov<0x101>((int) (pk >> 32));
    const uint64_t next = ((uint64_t) nhi << 32) | nlo;   // pick k + 1 (row_shl:1; K <= 16 keeps it in row 0)
    const uint32_t last = (uint32_t) __builtin_amdgcn_readlane((int) mk, K - 1);
    // tk[0] is now this lane's largest untaken key
    const bool bad = (lane + 1 < K && next != 0 && !(pk > next)) || last == 0u ||
                     (tk[0] & 0xFFFFFC00u) == (last & 0xFFFFFC00u);
    uint32_t mine = (uint32_t) (pk >> 32), myidx = pk ? pi : ~0u;
    if (__ballot(bad) != 0) {   // exact rounds on 64-bit keys: the maximum value, then the lowest index holding it
        uint64_t key[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) key[i] = pick_key(lv[i], lane + WAVE * i);
#pragma unroll
        for (int k = 2; k <= NV; k *= 2)
#pragma unroll
            for (int j = k / 2; j > 0; j /= 2)
#pragma unroll
                for (int i = 0; i < NV; ++i) {
                    const int l = i ^ j;
                    if (l > i) {
                        const bool desc = (i & k) == 0;
                        const uint64_t a = key[i], b = key[l];
                        const bool sw = desc ? a < b : a > b;
                        key[i] = sw ? b : a;
                        key[l] = sw ? a : b;
                    }
                }
        uint32_t ord[NV], idx[NV];   // an empty slot: ord 0, index ~0
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            ord[i] = (uint32_t) (key[i] >> 32);
            idx[i] = ~(uint32_t) key[i];
        }
        mine = 0;
        myidx = ~0u;
        for (int k = 0; k < K; ++k) {
            const uint32_t best = wave_max_u32(ord[0]);
            const uint32_t wi = wave_min_u32(ord[0] == best ? idx[0] : ~0u);
            if (lane == k) {
                mine = best;
                myidx = wi;
            }
            const bool won = idx[0] == wi;
#pragma unroll
            for (int i = 0; i + 1 < NV; ++i) {
                ord[i] = won ? ord[i + 1] : ord[i];
                idx[i] = won ? idx[i + 1] : idx[i];
            }
            ord[NV - 1] = won ? 0u : ord[NV - 1];
            idx[NV - 1] = won ? ~0u : idx[NV - 1];
        }
    }
    pick = mine ? (int) myidx : -1;
    pord = mine;
}
// the weights of the picks topk_picks returned (pord: the pick's value as order bits, 0 for none)
__device__ inline float topk_weight(int pick, uint32_t pord, int K) {
    const float myv = key_value((uint64_t) pord << 32);
    const float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(myv), 0));
    const float ek = pick >= 0 ? expf(myv - v0) : 0.f;
    float z = 0.f;
    for (int k = 0; k < K; ++k) z += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ek), k));
    return pick < 0 ? 0.f : ek / z;
}
template <int NV>
__device__ inline void topk_core(const float (&lv)[NV], int K, int lane, int& pick, float& weight) {
    uint32_t po;
    topk_picks<NV>(lv, K, lane, pick, po);
    weight = topk_weight(pick, po, K);
}

// AGENT: the logits were written earlier in the same launch
template <int NV, bool AGENT = false>
__device__ inline void topk_wave(const float* lg, int nv, int K, int lane, int& pick, float& weight) {
    float lv[NV];
    topk_load<NV, AGENT>(lg, nv, lane, lv);
    topk_core<NV>(lv, K, lane, pick, weight);
}
// E at run time (a multiple of 64, at most 1024): the smallest instantiation that holds E / 64 values a lane
template <bool AGENT = false>
__device__ inline void topk_wave_e(const float* lg, int E, int K, int lane, int& pick, float& weight) {
    const int nv = E / WAVE;
    if (nv <= 1) topk_wave<1, AGENT>(lg, nv, K, lane, pick, weight);
    else if (nv <= 2) topk_wave<2, AGENT>(lg, nv, K, lane, pick, weight);
    else if (nv <= 4) topk_wave<4, AGENT>(lg, nv, K, lane, pick, weight);
    else if (nv <= 8) topk_wave<8, AGENT>(lg, nv, K, lane, pick, weight);
    else topk_wave<16, AGENT>(lg, nv, K, lane, pick, weight);
}

// Decode jobs (src/moe.cuh:164-198, tools/kbench.cu:77-95): one job per distinct expert numbered in the order of each
// expert's first pick, a job's rows in pair order.  Thread p < P (one per pick, blockDim.x >= P) learns its pick's
// expert, its slot among the earlier picks of that expert, the expert's pick count and its job; returns the number of
// routed jobs.  ex: the picks (LDS); first: P bytes of LDS; jobof: E ints of LDS.
struct PickSlot {
    int e = -1, slot = 0, cnt = 0, job = -1;
};
// Each pick's slot in its expert's job: its rank among the picks of that expert (pair order), the job's row count, and
// the job's index (jobs numbered by first pick, pair order).  A row picks an expert at most once, so an expert's picks
// are told apart by their rows: a bit per row (T <= 32) in rows[e], the slot the bits below the pick's row.  The
// first picks are numbered by wavefront ballots.  Every thread of the block calls it (three barriers); the block holds
// at least P <= MAX_P threads; rows: MAX_E words of LDS, wsum: MAX_P / 64 ints of LDS.  Returns the number of jobs.
__device__ inline int pick_slots(const int* ex, int P, int K, unsigned* rows, int* jobof, int* wsum, PickSlot& ps) {
    const int p = threadIdx.x, lane = p % WAVE, wv = p / WAVE;
    ps = PickSlot{};
    const int e = p < P ? ex[p] : -1;
    if (e >= 0) rows[e] = 0u;
    __syncthreads();
    if (e >= 0) atomicOr(&rows[e], 1u << (p / K));
    __syncthreads();
    bool first = false;
    if (e >= 0) {
        const unsigned m = rows[e];
        ps.e = e;
        ps.slot = __popc(m & ((1u << (p / K)) - 1u));
        ps.cnt = __popc(m);
        first = ps.slot == 0;
    }
    const unsigned long long b = __ballot(first);
    if (lane == 0 && wv < MAX_P / WAVE) wsum[wv] = __popcll(b);
    __syncthreads();
    int off = 0, n = 0;
    for (int w = 0; w * WAVE < P; ++w) {
        off += w < wv ? wsum[w] : 0;
        n += wsum[w];
    }
    if (first) jobof[e] = off + __popcll(b & ((1ull << lane) - 1ull));
    __syncthreads();
    if (e >= 0) ps.job = jobof[e];
    return n;
}

}  // namespace sfnx
