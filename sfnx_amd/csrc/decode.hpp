// Decode internals: the workspace layout and each expert type's row of dot lanes.
#pragma once
#include "mv.hpp"
#include "topk.hpp"

namespace sfnx {

template <int TYPE> constexpr int lpr_of() { return is_kquant(TYPE) ? 8 : 16; }

struct DecLayout {
    size_t logits, xq, topi, topw, jg, jd, njobs, gu, hq_q, hq_d, hq_s, y, route_x, total;
};
// Every piece is laid out for the largest window (SFNX_MAXT rows), so the offsets are the same whatever T a call
// runs: a workspace sized once serves windows of any size, and a piece's row t always starts at t times its row size.
inline DecLayout dec_layout(int H, int E, int K, int ff) {
    constexpr int T = SFNX_MAXT;
    const size_t P = (size_t) T * K, NP = P + T, nj = P + 1;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t r = o;
        o += (bytes + 255) / 256 * 256;
        return r;
    };
    DecLayout L;
    L.logits = take((size_t) T * (E + 1) * 4);
    L.xq = take((size_t) T * (H / 32) * Q81_BYTES);
    L.topi = take(P * 4);
    L.topw = take(P * 4);
    L.jg = take(nj * sizeof(sfnx_job));
    L.jd = take(nj * sizeof(sfnx_job));
    L.njobs = take(8);
    L.gu = take(NP * 2 * ff * 4);
    L.hq_q = take(NP * ff);
    L.hq_d = take(NP * (ff / 32) * 4);
    L.hq_s = take(NP * (ff / 32) * 4);
    L.y = take((size_t) T * H * 4);
    L.route_x = take((size_t) XCDS * 2 * MAX_K * 4);   // batch 1: the picks and weights, a copy an XCD
    L.total = o;
    return L;
}

template <int TYPE, int G> struct RowOf;
template <int G> struct RowOf<SFNX_Q4_K, G> {
    using R = Q4kRow<G>;
    static __device__ __forceinline__ void load(R& w, const uint8_t* mat, int nrows, int row, int C, int ln) {
        w.load(q4k_planes(mat, nrows, C), row, C, ln);
    }
    static __device__ __forceinline__ void issue(R& w, const uint8_t* mat, int nrows, int row, int C, int ln) {
        w.issue(q4k_planes(mat, nrows, C), row, C, ln);
    }
};
template <int G> struct RowOf<SFNX_Q5_K, G> {
    using R = Q4kRow<G, true>;
    static __device__ __forceinline__ void load(R& w, const uint8_t* mat, int nrows, int row, int C, int ln) {
        w.load(q5k_planes(mat, nrows, C), row, C, ln);
    }
    static __device__ __forceinline__ void issue(R& w, const uint8_t* mat, int nrows, int row, int C, int ln) {
        w.issue(q5k_planes(mat, nrows, C), row, C, ln);
    }
};
template <int G> struct RowOf<SFNX_Q4_0, G> {
    using R = NbRow<G, SFNX_Q4_0>;
    static __device__ __forceinline__ void load(R& w, const uint8_t* mat, int nrows, int row, int C, int ln) {
        w.load(nb_planes<SFNX_Q4_0>(mat, nrows, C), row, C, ln);
    }
    static __device__ __forceinline__ void issue(R& w, const uint8_t* mat, int nrows, int row, int C, int ln) {
        w.issue(nb_planes<SFNX_Q4_0>(mat, nrows, C), row, C, ln);
    }
};
template <int G> struct RowOf<SFNX_Q5_1, G> {
    using R = NbRow<G, SFNX_Q5_1>;
    static __device__ __forceinline__ void load(R& w, const uint8_t* mat, int nrows, int row, int C, int ln) {
        w.load(nb_planes<SFNX_Q5_1>(mat, nrows, C), row, C, ln);
    }
    static __device__ __forceinline__ void issue(R& w, const uint8_t* mat, int nrows, int row, int C, int ln) {
        w.issue(nb_planes<SFNX_Q5_1>(mat, nrows, C), row, C, ln);
    }
};
template <int G> struct RowOf<SFNX_Q8_0, G> {
    using R = Q80Row<G>;
    static __device__ __forceinline__ void load(R& w, const uint8_t* mat, int nrows, int row, int C, int ln) {
        w.load(q80_planes(mat, nrows, C), row, C, ln);
    }
    static __device__ __forceinline__ void issue(R& w, const uint8_t* mat, int nrows, int row, int C, int ln) {
        w.issue(q80_planes(mat, nrows, C), row, C, ln);
    }
};


}  // namespace sfnx
