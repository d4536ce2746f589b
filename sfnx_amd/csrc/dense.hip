// The shared expert as the reference runs it when the model holds it as dense Q8_0 matrices (src/engine.cu:936-945):
// q8s_gemv of the q8_1 activations through gate|up, swiglu_stacked_q8_1, q8s_gemv of h through down into part rows
// P + t.  The dot is the reference's q8s sum (src/dense.cuh:24-154), here with 32 lanes a row as there; the fused
// decode computes the same sums on its own lane groups (q8s_dot in mv.hpp).  On the prompt path the reference runs its
// dense matrices as f16 GEMMs of the dequantized rows (pf_dense_xh): sfnx_pf_dense, on the matrix-core expert kernels
// (moe_mma.hip).
#include "mv.hpp"

namespace sfnx {
namespace {

constexpr int QS_THREADS = 256, QS_LPR = 32, QS_ROWS = QS_THREADS / QS_LPR, QS_TT = 4;

// a block of QS_ROWS rows; the activation rows staged QS_TT at a time: q8_1 rows y, or (SWIGLU) silu(gate) * up of the
// f32 rows y = [T][gate (cols) | up (cols)] quantized to q8_1 as they are staged (the same values as
// swiglu_stacked_q8_1's blocks, so the same sums as that call followed by q8s_gemv)
template <bool SWIGLU>
__global__ void __launch_bounds__(QS_THREADS) k_q8s_gemv(Q8sPlanes P, int rows, int cols, const uint8_t* __restrict__ y,
                                                        float* __restrict__ out, int out_stride, int T) {
    extern __shared__ __align__(16) unsigned char lds[];
    const Acts a = acts_in(lds, QS_TT, cols);
    const int row = blockIdx.x * QS_ROWS + threadIdx.x / QS_LPR, ln = threadIdx.x % QS_LPR;
    for (int t0 = 0; t0 < T; t0 += QS_TT) {
        const int nn = min(QS_TT, T - t0);
        if (t0) __syncthreads();
        if constexpr (SWIGLU) stage_swiglu(a, reinterpret_cast<const float*>(y) + (size_t) t0 * 2 * cols, nullptr, nn);
        else stage_q8_1(a, y + (size_t) t0 * (cols / 32) * Q81_BYTES, nullptr, nn);
        __syncthreads();
        for (int j = 0; j < nn; ++j) {
            const float v = group_sum<QS_LPR>(row < rows ? q8s_dot<QS_LPR>(P, row, cols, ln, a, j) : 0.f);
            if (row < rows && ln == 0) out[(size_t) (t0 + j) * out_stride + row] = v;
        }
    }
}

// src/kernels.cu:1948-1963 k_swiglu_stacked: a half-wave per (row t, 32 values)
__global__ void k_swiglu_stacked(const float* __restrict__ gu, uint8_t* __restrict__ hq, int ffs, int T) {
    const int t = blockIdx.y, b = blockIdx.x * (blockDim.x / 32) + threadIdx.x / 32, l = threadIdx.x % 32;
    if (b >= ffs / 32) return;   // whole half-waves leave together
    const float* g = gu + (size_t) t * 2 * ffs;
    const float xi = silu_f(g[32 * b + l]) * g[ffs + 32 * b + l];
    const float amax = group_max<32>(fabsf(xi)), sum = group_sum<32>(xi);
    const float d = amax / 127.0f;
    uint8_t* blk = hq + ((size_t) t * (ffs / 32) + b) * Q81_BYTES;
    blk[4 + l] = (uint8_t) (int8_t) (amax == 0.0f ? 0 : (int) roundf(xi / d));
    if (l == 0) *reinterpret_cast<uint32_t*>(blk) = (uint32_t) f2h(d) | ((uint32_t) f2h(sum) << 16);
}

// src/model.cpp:384-440 q8split: GGUF Q8_0 blocks into the split planes, a thread a block
__global__ void k_q8s_split(const uint8_t* __restrict__ blocks, int rows, int cols, int8_t* __restrict__ q,
                            uint16_t* __restrict__ d) {
    const int nb = cols / 32;
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t) rows * nb) return;
    const uint8_t* b = blocks + i * Q80_BYTES;
    d[i] = (uint16_t) (b[0] | (b[1] << 8));
    int4* dst = reinterpret_cast<int4*>(q + i * 32);
    int w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = b[2 + 4 * k] | (b[3 + 4 * k] << 8) | (b[4 + 4 * k] << 16) | (b[5 + 4 * k] << 24);
    dst[0] = make_int4(w[0], w[1], w[2], w[3]);
    dst[1] = make_int4(w[4], w[5], w[6], w[7]);
}

// the split planes into the planar Q8_0 layout of one matrix (the matrix-core kernels' operand), a thread a block:
// its two 16-value halves to their pieces, its scale to the scale plane
__global__ void k_q8s_to_planar(Q8sPlanes W, int rows, int cols, uint8_t* __restrict__ dst) {
    const int nb = cols / 32;
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t) rows * nb) return;
    const int r = (int) (i / nb), b = (int) (i % nb);
    const Q80Planes P = q80_planes(dst, rows, cols);
#pragma unroll
    for (int h = 0; h < 2; ++h)
        *reinterpret_cast<int4*>(const_cast<uint8_t*>(P.q16(r, cols, 32 * (b / 16) + 16 * h + b % 16))) =
            *reinterpret_cast<const int4*>(W.q16(r, cols, 32 * b + 16 * h));
    *const_cast<uint16_t*>(P.dof(r, cols, b)) = *W.dof(r, cols, b);
}

}  // namespace

// bytes of one matrix's planar Q8_0 staging (rows x cols values)
size_t q8s_planar_bytes(int rows, int cols) { return (size_t) rows * row_bytes(SFNX_Q8_0, cols); }
void q8s_to_planar(const sfnx_q8s& W, int rows, int cols, void* dst, hipStream_t s) {
    const size_t n = (size_t) rows * (cols / 32);
    k_q8s_to_planar<<<(unsigned) ((n + 255) / 256), 256, 0, s>>>(Q8sPlanes{W.q, W.d}, rows, cols, (uint8_t*) dst);
}
}  // namespace sfnx

using namespace sfnx;

extern "C" int sfnx_q8s_gemv(const sfnx_q8s* W, int rows, int cols, const void* y, float* out, int out_stride, int T,
                             void* st) {
    return guarded("sfnx_q8s_gemv", [&] {
        require(W != nullptr && W->q != nullptr && W->d != nullptr && y != nullptr && out != nullptr, "null pointer");
        require(rows > 0 && rows % 32 == 0, "rows must be a positive multiple of 32");
        require(cols > 0 && cols % 512 == 0, "cols must be a positive multiple of 512");
        require(T >= 1 && T <= 65535, "T out of range");
        require(out_stride >= rows, "out_stride smaller than rows");
        const size_t lds = acts_bytes(QS_TT, cols);
        require(lds <= 64 * 1024, "cols too wide for the activation staging");
        k_q8s_gemv<false><<<(rows + QS_ROWS - 1) / QS_ROWS, QS_THREADS, lds, stream_of(st)>>>(
            Q8sPlanes{W->q, W->d}, rows, cols, (const uint8_t*) y, out, out_stride, T);
    });
}

extern "C" int sfnx_q8s_swiglu_gemv(const sfnx_q8s* W, int rows, int ffs, const float* gu, float* out, int out_stride,
                                    int T, void* st) {
    return guarded("sfnx_q8s_swiglu_gemv", [&] {
        require(W != nullptr && W->q != nullptr && W->d != nullptr && gu != nullptr && out != nullptr, "null pointer");
        require(rows > 0 && rows % 32 == 0, "rows must be a positive multiple of 32");
        require(ffs > 0 && ffs % 512 == 0, "ffs must be a positive multiple of 512");
        require(T >= 1 && T <= 65535, "T out of range");
        require(out_stride >= rows, "out_stride smaller than rows");
        const size_t lds = acts_bytes(QS_TT, ffs);
        require(lds <= 64 * 1024, "ffs too wide for the activation staging");
        k_q8s_gemv<true><<<(rows + QS_ROWS - 1) / QS_ROWS, QS_THREADS, lds, stream_of(st)>>>(
            Q8sPlanes{W->q, W->d}, rows, ffs, (const uint8_t*) gu, out, out_stride, T);
    });
}

extern "C" int sfnx_swiglu_stacked_q8_1(const float* gu, void* hq, int ffs, int T, void* st) {
    return guarded("sfnx_swiglu_stacked_q8_1", [&] {
        require(gu != nullptr && hq != nullptr, "null pointer");
        require(ffs > 0 && ffs % 32 == 0, "ffs must be a positive multiple of 32");
        require(T >= 1 && T <= 65535, "T out of range");
        const dim3 grid((ffs / 32 + 7) / 8, T);
        k_swiglu_stacked<<<grid, 256, 0, stream_of(st)>>>(gu, (uint8_t*) hq, ffs, T);
    });
}

extern "C" int sfnx_q8s_split(const void* blocks, int rows, int cols, const sfnx_q8s* W, void* st) {
    return guarded("sfnx_q8s_split", [&] {
        require(blocks != nullptr && W != nullptr && W->q != nullptr && W->d != nullptr, "null pointer");
        require(rows > 0 && cols > 0 && cols % 32 == 0, "rows must be positive and cols a positive multiple of 32");
        const size_t n = (size_t) rows * (cols / 32);
        k_q8s_split<<<(unsigned) ((n + 255) / 256), 256, 0, stream_of(st)>>>((const uint8_t*) blocks, rows, cols, W->q, W->d);
    });
}
