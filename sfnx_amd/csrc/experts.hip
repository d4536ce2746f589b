// The routed experts as grouped matrix x few-vectors products on int8 dot instructions (v_dot4_i32_i8): gate|up of
// the q8_1 activations, and down of h = silu(gate) * up quantized to q8_1 in LDS.  One launch covers every job of a
// layer: blockIdx.y is the job, blockIdx.x a tile of the expert's rows.  A job's activations are staged in LDS once;
// each lane keeps its share of a weight row in registers across the job's rows (several passes for BigJobs).
//
// Arithmetic per (row, activation row), identical to the CPU oracle's:
//   Q4_K: 8 lanes a row, lane l8 the 64-value groups l8 + 8 i in order (src/moe_q4k.cuh:30-86), each group
//         d (d8l (sc0 dl) + d8h (sc1 dh)) - dmin (d8l (m0 sl) + d8h (m1 sh)), then xor 4, 2, 1 (src/moe.cuh:224-235).
//   Q5_K: as Q4_K on the 5-bit values.
//   Q4_0 / Q5_1: the Q8_0 lanes; per block (d_w d_a) sum (q - 8) a, or (d_w d_a) sum q a + (m_w d_a) sum a.
//   Q8_0: 16 lanes a row, lane l16 the 32-blocks l16 + 16 i in order, each (d_w d_a) sum(q_w q_a), then xor 8 .. 1.
#include <type_traits>

#include "mv.hpp"

namespace sfnx {
namespace {

constexpr int MV_THREADS = 256;
#ifndef MV_THREADS_DOWN
#define MV_THREADS_DOWN 1024
#endif
#ifndef MV_RPL_DOWN
#define MV_RPL_DOWN 4
#endif

// The prompt path's BigJobs (up to 64 activation rows a job): down of FF 512 on 1024-thread workgroups, 4 rows a lane
// group, so the job's h (recomputed from gate|up by every workgroup while staging it) is computed by a sixteenth as
// many workgroups, and each activation read serves 4 rows.  Decode windows (a few rows a job, few jobs) keep 256
// threads and a row a lane group, for their parallelism.
constexpr bool mv_big_down(uint32_t type, int G, bool down, bool big) { return big && down && G == 1 && type != SFNX_Q8_0; }
template <int TYPE, int G, bool DOWN, bool BIG> constexpr int mv_threads() {
    return mv_big_down(TYPE, G, DOWN, BIG) ? MV_THREADS_DOWN : MV_THREADS;
}
template <int TYPE, int G, bool DOWN, bool BIG> constexpr int mv_rows_per_lane() {
    return mv_big_down(TYPE, G, DOWN, BIG) ? MV_RPL_DOWN : 1;
}

// ------------------------------------------------------------------------------------------------ the kernel
// TYPE: SFNX_Q4_K / SFNX_Q5_K (8 lanes a row) or SFNX_Q8_0 (16 lanes a row); G: groups or blocks per lane = C / 512;
// TT: activation rows per pass; DOWN: activations from gu rows through swiglu (else q8_1 rows).
template <int TYPE, int G, int TT, bool DOWN, typename J>
__global__ void __launch_bounds__((mv_threads<TYPE, G, DOWN, std::is_same_v<J, sfnx_bigjob>>()))
k_moe_mv(const uint8_t* __restrict__ A, size_t sa, int R, int C, const J* __restrict__ jobs, const int* __restrict__ njobs,
         const void* __restrict__ in, float* __restrict__ out) {
    constexpr bool BIG = std::is_same_v<J, sfnx_bigjob>;
    constexpr int LPR = is_kquant(TYPE) ? 8 : 16, RPB = mv_threads<TYPE, G, DOWN, BIG>() / LPR;
    constexpr int RPL = mv_rows_per_lane<TYPE, G, DOWN, BIG>();
    // the last job first: with a shared expert it is the shared one, which holds every row of the window (or, on the
    // prompt path, a run of full 64-row jobs); dispatched last, its blocks ran alone at the launch's end
    const int nj = *njobs;
    if ((int) blockIdx.y >= nj) return;
    const int ji = ((int) blockIdx.y + nj - 1) % nj;
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ J jb;
    load_job(jb, jobs + ji);
    __syncthreads();
    const int row = blockIdx.x * RPB * RPL + threadIdx.x / LPR, ln = threadIdx.x % LPR;   // (and row + RPB r, r < RPL)
    const bool live = row < R;
    const uint8_t* mat = expert_at(A, sa, jb.w);
    const Acts a = acts_in(lds, TT, C);
    if constexpr (TYPE != SFNX_Q8_0) {
        using Row = std::conditional_t<is_kquant(TYPE), Q4kRow<G, TYPE == SFNX_Q5_K>, NbRow<G, TYPE>>;
        Row w[RPL];
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const int rr = row + RPB * r;
            if constexpr (is_kquant(TYPE)) {
                if (rr < R) w[r].load(kq_planes<TYPE == SFNX_Q5_K>(mat, R, C), rr, C, ln);
            } else {
                if (rr < R) w[r].load(nb_planes<TYPE>(mat, R, C), rr, C, ln);
            }
        }
        for (int j0 = 0; j0 < jb.n; j0 += TT) {
            const int nn = min(TT, jb.n - j0);
            if (j0) __syncthreads();
            if constexpr (DOWN) stage_swiglu(a, (const float*) in, jb.y + j0, nn);
            else stage_q8_1(a, (const uint8_t*) in, jb.y + j0, nn);
            __syncthreads();
            for (int j = 0; j < nn; ++j) {
                float v[RPL];
#pragma unroll
                for (int r = 0; r < RPL; ++r) v[r] = group_sum<LPR>(row + RPB * r < R ? w[r].dot(a, j, ln) : 0.f);
                if (ln == 0)
#pragma unroll
                    for (int r = 0; r < RPL; ++r)
                        if (row + RPB * r < R) out[(size_t) jb.out[j0 + j] * R + row + RPB * r] = v[r];
            }
        }
    } else {
        Q80Row<G> w;
        if (live) w.load(q80_planes(mat, R, C), row, C, ln);
        for (int j0 = 0; j0 < jb.n; j0 += TT) {
            const int nn = min(TT, jb.n - j0);
            if (j0) __syncthreads();
            if constexpr (DOWN) stage_swiglu(a, (const float*) in, jb.y + j0, nn);
            else stage_q8_1(a, (const uint8_t*) in, jb.y + j0, nn);
            __syncthreads();
            for (int j = 0; j < nn; ++j) {
                const float v = group_sum<LPR>(live ? w.dot(a, j, ln) : 0.f);
                if (live && ln == 0) out[(size_t) jb.out[j0 + j] * R + row] = v;
            }
        }
    }
}

template <int TYPE, int TT, bool DOWN, typename J>
void launch_g(int G, dim3 grid, size_t lds, hipStream_t s, const uint8_t* A, size_t sa, int R, int C, const J* jobs,
              const int* njobs, const void* in, float* out) {
    constexpr bool BIGJ = std::is_same_v<J, sfnx_bigjob>;
    switch (G) {
        case 1: k_moe_mv<TYPE, 1, TT, DOWN, J><<<grid, mv_threads<TYPE, 1, DOWN, BIGJ>(), lds, s>>>(A, sa, R, C, jobs, njobs, in, out); break;
        case 2: k_moe_mv<TYPE, 2, TT, DOWN, J><<<grid, mv_threads<TYPE, 2, DOWN, BIGJ>(), lds, s>>>(A, sa, R, C, jobs, njobs, in, out); break;
        case 4: k_moe_mv<TYPE, 4, TT, DOWN, J><<<grid, mv_threads<TYPE, 4, DOWN, BIGJ>(), lds, s>>>(A, sa, R, C, jobs, njobs, in, out); break;
        case 5: k_moe_mv<TYPE, 5, TT, DOWN, J><<<grid, mv_threads<TYPE, 5, DOWN, BIGJ>(), lds, s>>>(A, sa, R, C, jobs, njobs, in, out); break;
        case 8: k_moe_mv<TYPE, 8, TT, DOWN, J><<<grid, mv_threads<TYPE, 8, DOWN, BIGJ>(), lds, s>>>(A, sa, R, C, jobs, njobs, in, out); break;
        default: throw std::runtime_error("input width must be 512, 1024, 2048, 2560 or 4096");
    }
}

template <bool DOWN, typename J>
void moe_mv(uint32_t type, const void* A, size_t sa, int n_in, int n_out, const J* jobs, const int* njobs, int njobs_max,
            int T, const void* in, float* out, void* st) {
    require(expert_type_ok(type), TYPE_MSG);
    require(n_in > 0 && n_in % 512 == 0, "expert input width must be a multiple of 512");
    require(n_out > 0, "expert rows must be positive");
    require(stride_ok(sa, row_bytes(type, n_in) * (size_t) n_out), "expert stride smaller than a matrix");
    require(njobs_max >= 0 && njobs_max <= 65535, "njobs_max out of range");
    if (njobs_max == 0) return;
    const int G = n_in / 512;
    // activation rows staged per pass: up to 16 while they fit 64 KiB of LDS (the kernel loops over the passes)
    int TT = T <= 1 ? 1 : T <= 4 ? 4 : 16;
    if (acts_bytes(TT, n_in) > 64 * 1024) TT = 4;
    const size_t lds = acts_bytes(TT, n_in);
    require(lds <= 64 * 1024, "activation rows do not fit the LDS budget");
    const bool bd = mv_big_down(type, G, DOWN, std::is_same_v<J, sfnx_bigjob>);
    const int rpb = (bd ? MV_THREADS_DOWN : MV_THREADS) / (is_kquant(type) ? 8 : 16) * (bd ? MV_RPL_DOWN : 1);
    const dim3 grid((n_out + rpb - 1) / rpb, njobs_max);
    hipStream_t s = stream_of(st);
    const uint8_t* a = (const uint8_t*) A;
#define SFNX_MV(TY, TTV) launch_g<TY, TTV, DOWN, J>(G, grid, lds, s, a, sa, n_out, n_in, jobs, njobs, in, out)
    if (type == SFNX_Q4_K) {
        if (TT == 1) SFNX_MV(SFNX_Q4_K, 1);
        else if (TT == 4) SFNX_MV(SFNX_Q4_K, 4);
        else SFNX_MV(SFNX_Q4_K, 16);
    } else if (type == SFNX_Q5_K) {
        if (TT == 1) SFNX_MV(SFNX_Q5_K, 1);
        else if (TT == 4) SFNX_MV(SFNX_Q5_K, 4);
        else SFNX_MV(SFNX_Q5_K, 16);
    } else if (type == SFNX_Q4_0) {
        if (TT == 1) SFNX_MV(SFNX_Q4_0, 1);
        else if (TT == 4) SFNX_MV(SFNX_Q4_0, 4);
        else SFNX_MV(SFNX_Q4_0, 16);
    } else if (type == SFNX_Q5_1) {
        if (TT == 1) SFNX_MV(SFNX_Q5_1, 1);
        else if (TT == 4) SFNX_MV(SFNX_Q5_1, 4);
        else SFNX_MV(SFNX_Q5_1, 16);
    } else {
        if (TT == 1) SFNX_MV(SFNX_Q8_0, 1);
        else if (TT == 4) SFNX_MV(SFNX_Q8_0, 4);
        else SFNX_MV(SFNX_Q8_0, 16);
    }
#undef SFNX_MV
}

}  // namespace
}  // namespace sfnx

using namespace sfnx;

extern "C" int sfnx_moe_gate_up(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_job* jobs,
                                const int* njobs, int njobs_max, int T, const void* xq, float* gu, void* st) {
    return guarded("sfnx_moe_gate_up", [&] {
        require(T >= 1 && T <= SFNX_MAXT, "T out of range (1..16)");
        moe_mv<false>(type, A, sa, n_in, n_out, jobs, njobs, njobs_max, T, xq, gu, st);
    });
}

extern "C" int sfnx_moe_down(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_job* jobs,
                             const int* njobs, int njobs_max, int T, const float* gu, float* part, void* st) {
    return guarded("sfnx_moe_down", [&] {
        require(T >= 1 && T <= SFNX_MAXT, "T out of range (1..16)");
        moe_mv<true>(type, A, sa, n_in, n_out, jobs, njobs, njobs_max, T, gu, part, st);
    });
}

extern "C" int sfnx_moe_gate_up_big(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_bigjob* jobs,
                                    const int* njobs, int njobs_cap, const void* xq, float* gu, void* st) {
    return guarded("sfnx_moe_gate_up_big", [&] { moe_mv<false>(type, A, sa, n_in, n_out, jobs, njobs, njobs_cap, SFNX_PF_JOB, xq, gu, st); });
}

extern "C" int sfnx_moe_down_big(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_bigjob* jobs,
                                 const int* njobs, int njobs_cap, const float* gu, float* part, void* st) {
    return guarded("sfnx_moe_down_big", [&] { moe_mv<true>(type, A, sa, n_in, n_out, jobs, njobs, njobs_cap, SFNX_PF_JOB, gu, part, st); });
}
