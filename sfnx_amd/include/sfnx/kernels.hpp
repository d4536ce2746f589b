// C++ face of libsfnx_moe.so under the reference engine's names (src/kernels.hpp:18-36, 269-313): the calls an engine
// makes for its MoE half, each a thin inline wrapper over the C ABI (include/sfnx_moe.h) that throws
// std::runtime_error with the library's message on failure, as the reference's wrappers do (src/kernels.cu:31-34).
//
// The reference fixes the hidden size, expert count and top-k at compile time (src/model.hpp:40-45: N, NEXP, TOPK);
// here they are a runtime MoeShape.  The weights are the planar store (sfnx_store_pack) rather than raw GGUF rows.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>

#include "sfnx_moe.h"

namespace sfnx {

using Job = sfnx_job;         // src/kernels.hpp:18-23
using BigJob = sfnx_bigjob;   // src/kernels.hpp:25-32
constexpr int MAXT = SFNX_MAXT, PF_JOB = SFNX_PF_JOB;
enum GgmlType : uint32_t {   // src/gguf.hpp:22-25
    T_Q4_0 = SFNX_Q4_0, T_Q5_1 = SFNX_Q5_1, T_Q8_0 = SFNX_Q8_0, T_Q4_K = SFNX_Q4_K, T_Q5_K = SFNX_Q5_K
};

// src/model.hpp:71-74 Q8S: a dense Q8_0 matrix in the split layout, int8 values q [rows][cols] and f16 scale bits
// d [rows][cols / 32] (the C struct, so the reference's fields and their types)
using Q8S = sfnx_q8s;

// src/model.hpp:78-87 DW: one matrix (or expert 0's of a stack), n_out rows of n_in.  row_bytes and s are kept for
// the reference's field list (row_bytes is derived from type and n_in here; s is the dense form of a matrix).  ep: a
// device table of each expert's matrix (the reference's expert-cache tables); when set, the calls pass it across the C
// boundary as the store with stride 0, and the stride argument is unused, as in moe_expert (src/moe_w.cuh:9).
struct DW {
    const void* p = nullptr;
    uint32_t type = 0;
    int n_in = 0, n_out = 0;
    size_t row_bytes = 0;
    Q8S s;
    const char* const* ep = nullptr;
};
namespace detail {
// a DW's experts at the C boundary: the pointer table (stride 0) when ep is set, else p and the stride
inline const void* base_of(const DW& A) { return A.ep ? static_cast<const void*>(A.ep) : A.p; }
inline size_t stride_of(const DW& A, size_t sa) { return A.ep ? 0 : sa; }
}  // namespace detail

// the sizes the reference compiles in
struct MoeShape {
    int H = 2048;    // N
    int E = 512;     // NEXP
    int K = 10;      // TOPK
};

// The reference fixes N, NEXP and TOPK at compile time (src/model.hpp:40-45), so its calls do not pass them.  The
// overloads below that keep the reference's argument lists exactly read them from here: set once, before the first
// call, as the reference's build fixes them.  (The overloads that take a MoeShape are the same calls with the shape
// passed explicitly.)
inline MoeShape& model_shape() {
    static MoeShape s;
    return s;
}
inline void set_model_shape(const MoeShape& s) { model_shape() = s; }

// src/model.hpp:95-116 ExpertCache (routed experts kept in host RAM, VRAM slots for the ones in use): the C struct,
// whose fields keep the reference's names (its arena fields, slots lent to a K/V pool, have no counterpart)
using ExpertCache = sfnx_expert_cache;

inline void ck(int status) {
    if (status != 0) throw std::runtime_error(sfnx_last_error());
}

constexpr size_t q8_1_bytes(int n) { return (size_t) (n / 32) * 36; }   // src/kernels.hpp:34

inline void quantize_q8_1(const float* x, void* q, int n, int rows, void* st) { ck(sfnx_quantize_q8_1(x, q, n, rows, st)); }


// src/kernels.hpp:47 (src/dense.cuh:24-154): the shared expert's dense Q8_0 product in the reference's q8s sums
inline void q8s_gemv(const Q8S& w, int rows, int cols, const void* y, float* out, int out_stride, int T, void* st) {
    ck(sfnx_q8s_gemv(&w, rows, cols, y, out, out_stride, T, st));
}
// src/kernels.cu:2018-2024
inline void swiglu_stacked_q8_1(const float* gu, void* hq, int ffs, int T, void* st) { ck(sfnx_swiglu_stacked_q8_1(gu, hq, ffs, T, st)); }

// src/kernels.hpp:276-278; shared: the shared expert (expert E of the stacks) rides as the last job
inline void router_route(const MoeShape& s, const float* W, const float* x, float* logits, int T, int* topi, float* topw,
                         Job* jobs_gu, Job* jobs_dn, int* njobs, void* st, bool shared = true) {
    ck(sfnx_router_route(W, x, logits, T, s.H, s.E, s.K, topi, topw, jobs_gu, jobs_dn, njobs, shared ? 1 : 0, st));
}
// src/kernels.hpp:276-278 with the dense shared expert's gate|up (sh_gu: sh_rows = 2 ffs rows over the q8_1 rows
// sh_y into sh_out, row stride sh_rows).  The reference runs it in the router's launch; here it is sfnx_q8s_gemv after
// the routing on the same stream: the same q8s sums, so the same values.  The shared expert is then no routed job.
inline void router_route(const MoeShape& s, const float* W, const float* x, float* logits, int T, int* topi, float* topw,
                         Job* jobs_gu, Job* jobs_dn, int* njobs, void* st, const Q8S* sh_gu, int sh_rows, const void* sh_y,
                         float* sh_out) {
    router_route(s, W, x, logits, T, topi, topw, jobs_gu, jobs_dn, njobs, st, /*shared=*/false);
    if (sh_gu) q8s_gemv(*sh_gu, sh_rows, s.H, sh_y, sh_out, sh_rows, T, st);
}
// src/kernels.hpp:281-282; T: the window's rows (the reference derives it as njobs_max / TOPK)
inline void moe_gate_up(const DW& A, size_t sa, const Job* jobs, const int* njobs, int njobs_max, const void* xq, float* gu,
                        void* st, int T) {
    ck(sfnx_moe_gate_up(detail::base_of(A), detail::stride_of(A, sa), A.type, A.n_in, A.n_out, jobs, njobs, njobs_max, T, xq, gu, st));
}
// src/kernels.hpp:281-282 with the dense shared expert's SwiGLU and down (sh_down: N rows of sh_ffs; sh_gu [T][2 sh_ffs]
// into sh_out, row stride N).  The reference runs them in the gate|up launch; here sfnx_swiglu_stacked_q8_1 and
// sfnx_q8s_gemv follow on the same stream, with the same values.  sh_hq: the caller's [T][sh_ffs / 32] q8_1 rows for h
// (the reference keeps h in shared memory; a library call that allocates nothing needs the buffer from its caller).
inline void moe_gate_up(const DW& A, size_t sa, const Job* jobs, const int* njobs, int njobs_max, const void* xq, float* gu,
                        void* st, int T, const Q8S* sh_down, int sh_ffs, const float* sh_gu, float* sh_out, void* sh_hq) {
    moe_gate_up(A, sa, jobs, njobs, njobs_max, xq, gu, st, T);
    if (sh_down) {
        swiglu_stacked_q8_1(sh_gu, sh_hq, sh_ffs, T, st);
        q8s_gemv(*sh_down, A.n_in, sh_ffs, sh_hq, sh_out, A.n_in, T, st);
    }
}
// ------------------------------------------------------------------------------------------------ the reference's
// argument lists (src/kernels.hpp:276-305), N / NEXP / TOPK from model_shape().  As in the reference engine
// (src/engine.cu:933-978) the shared expert is no routed job here: it is the dense Q8_0 matrices passed through the
// sh_* arguments, and its rows are part rows T TOPK + t.
namespace detail {
inline void no_cache(const ExpertCache* ec, const DW* w = nullptr) {
    (void) ec;
    (void) w;
}
// the window's rows from the job grid's size, as the reference's moe_mm does (src/kernels.cu:1931)
inline int rows_of(int njobs_max) {
    const int T = njobs_max / model_shape().K;
    return T < 1 ? 1 : (T > MAXT ? MAXT : T);
}
}  // namespace detail

// src/kernels.hpp:276-278
inline void router_route(const float* W, const float* x, float* logits, int T, int* topi, float* topw, Job* jobs_gu,
                         Job* jobs_dn, int* njobs, void* st, const ExpertCache* ec = nullptr, int layer = -1,
                         int* list = nullptr, const Q8S* sh_gu = nullptr, int sh_rows = 0, const void* sh_y = nullptr,
                         float* sh_out = nullptr) {
    const MoeShape& s = model_shape();
    if (ec && (layer < 0 || !list)) throw std::runtime_error("router_route: a cache plan needs its layer and list");
    // with a cache, the router launch's last block plans the window's slots, as the reference's does
    if (ec) ck(sfnx_router_route_plan(W, x, logits, T, s.H, s.E, s.K, topi, topw, jobs_gu, jobs_dn, njobs, 0, ec, layer, list, st));
    else ck(sfnx_router_route(W, x, logits, T, s.H, s.E, s.K, topi, topw, jobs_gu, jobs_dn, njobs, 0, st));
    if (sh_gu) ck(sfnx_q8s_gemv(sh_gu, sh_rows, s.H, sh_y, sh_out, sh_rows, T, st));
}
// src/kernels.cu:1655-1668 cache_copy / moe_cache: the planned experts into their slots (moe_cache plans first when
// given the jobs)
inline void cache_copy(const ExpertCache& ec, int p, const int* list, void* st) { ck(sfnx_cache_copy(&ec, p, list, st)); }
inline void moe_cache(int layer, size_t gu_stride, size_t dn_stride, const ExpertCache& ec, int* list, void* st,
                      const Job* jobs = nullptr, const int* njobs = nullptr) {
    ck(sfnx_moe_cache(layer, gu_stride, dn_stride, &ec, list, jobs, njobs, st));
}
// src/kernels.hpp:281-282: the shared expert's SwiGLU and down (sh_down: N rows of sh_ffs) from sh_gu ([T][2 sh_ffs])
// into sh_out (row stride N), as the reference's fused launch computes them; T from njobs_max
inline void moe_gate_up(const DW& A, size_t sa, const Job* jobs, const int* njobs, int njobs_max, const void* xq, float* gu,
                        void* st, const Q8S* sh_down = nullptr, int sh_ffs = 0, const float* sh_gu = nullptr,
                        float* sh_out = nullptr) {
    detail::no_cache(nullptr, &A);
    const int T = detail::rows_of(njobs_max);
    ck(sfnx_moe_gate_up(detail::base_of(A), detail::stride_of(A, sa), A.type, A.n_in, A.n_out, jobs, njobs, njobs_max, T, xq, gu, st));
    if (sh_down) ck(sfnx_q8s_swiglu_gemv(sh_down, A.n_in, sh_ffs, sh_gu, sh_out, A.n_in, T, st));
}
// src/kernels.hpp:305
inline void moe_down(const DW& A, size_t sa, const Job* jobs, const int* njobs, int njobs_max, const float* gu, float* part,
                     void* st) {
    detail::no_cache(nullptr, &A);
    ck(sfnx_moe_down(detail::base_of(A), detail::stride_of(A, sa), A.type, A.n_in, A.n_out, jobs, njobs, njobs_max, detail::rows_of(njobs_max), gu, part, st));
}
// src/kernels.hpp:290-292: the prompt path's matrix-core calls (moe_mma.cuh)
inline void moe_gate_up_mma(const DW& A, size_t sa, const BigJob* jobs, const int* njobs, int njobs_cap, const uint16_t* xh,
                            float* gu, void* st) {
    detail::no_cache(nullptr, &A);
    ck(sfnx_moe_gate_up_mma(detail::base_of(A), detail::stride_of(A, sa), A.type, A.n_in, A.n_out, jobs, njobs, njobs_cap, xh, gu, st));
}
inline void swiglu_h16(const float* gu, int ffs, int P, uint16_t* h16, void* st) { ck(sfnx_swiglu_h16(gu, ffs, P, h16, st)); }
inline void moe_down_mma(const DW& A, size_t sa, const BigJob* jobs, const int* njobs, int njobs_cap, const uint16_t* h16,
                         float* part, void* st) {
    detail::no_cache(nullptr, &A);
    ck(sfnx_moe_down_mma(detail::base_of(A), detail::stride_of(A, sa), A.type, A.n_in, A.n_out, jobs, njobs, njobs_cap, h16, part, st));
}

// src/kernels.hpp:284: jobs of up to MAXT rows each, njobs_cap of them at most (the prompt path's)
inline void moe_gate_up_jobs(const DW& A, size_t sa, const Job* jobs, const int* njobs, int njobs_cap, const void* xq,
                             float* gu, void* st) {
    moe_gate_up(A, sa, jobs, njobs, njobs_cap, xq, gu, st, MAXT);
}
// src/kernels.hpp:305
inline void moe_down(const DW& A, size_t sa, const Job* jobs, const int* njobs, int njobs_max, const float* gu, float* part,
                     void* st, int T) {
    ck(sfnx_moe_down(detail::base_of(A), detail::stride_of(A, sa), A.type, A.n_in, A.n_out, jobs, njobs, njobs_max, T, gu, part, st));
}
// src/kernels.hpp:286-287
inline void moe_gate_up_big(const DW& A, size_t sa, const BigJob* jobs, const int* njobs, int njobs_cap, const void* xq,
                            float* gu, void* st) {
    ck(sfnx_moe_gate_up_big(detail::base_of(A), detail::stride_of(A, sa), A.type, A.n_in, A.n_out, jobs, njobs, njobs_cap, xq, gu, st));
}
inline void moe_down_big(const DW& A, size_t sa, const BigJob* jobs, const int* njobs, int njobs_cap, const float* gu,
                         float* part, void* st) {
    ck(sfnx_moe_down_big(detail::base_of(A), detail::stride_of(A, sa), A.type, A.n_in, A.n_out, jobs, njobs, njobs_cap, gu, part, st));
}
// the prompt path's routing (src/prefill.cu:1163-1167: router sgemm, k_pf_top10, k_pf_count, k_pf_jobbase, k_pf_fill)
inline void router_logits(const float* W, const float* x, float* logits, int T, int H, int L, void* st) {
    ck(sfnx_router_logits(W, x, logits, T, H, L, st));
}
inline void pf_route(const MoeShape& s, const float* logits, int C, int* topi, float* topw, int* cnt, int* jbase,
                     BigJob* jobs_gu, BigJob* jobs_dn, int* njobs, void* st, bool shared = true) {
    ck(sfnx_pf_route(logits, C, s.E, s.K, topi, topw, cnt, jbase, jobs_gu, jobs_dn, njobs, shared ? 1 : 0, st));
}
// the weighted combine the reference folds into its ring sum (src/kernels.cu:797-803, RingMoe src/kernels.hpp:309-313)
inline void moe_combine(const MoeShape& s, const float* part, const float* topw, const int* topi, const float* logits,
                        float* y, int T, void* st, bool shared = true) {
    ck(sfnx_moe_combine(part, topw, topi, logits, y, T, s.H, s.E, s.K, shared ? 1 : 0, st));
}

// src/kernels.cu:1054 hc_read: N, HC and LR are the reference's compile-time model constants (src/model.hpp:39);
// scratch is sfnx_hc_workspace(N, HC, LR) bytes (no barrier counter and no err word: no kernel waits on another)
inline void hc_read(float* R, const float* bo, const float* inj_prev, const float* w_norm, const Q8S& w_down,
                    const Q8S& w_up, const uint16_t* w_inj, float eps, float* mixed, float* inject, void* scratch,
                    size_t scratch_bytes, int T, void* st, void* q8, int N, int HC, int LR) {
    ck(sfnx_hc_read(R, bo, inj_prev, w_norm, w_down.q, w_down.d, w_up.q, w_up.d, w_inj, eps, mixed, inject, q8, T, N, HC,
                    LR, scratch, scratch_bytes, st));
}

static_assert(sizeof(Job) == 136 && sizeof(BigJob) == 520, "job layouts match the reference's");

}  // namespace sfnx
