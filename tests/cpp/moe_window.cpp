// A decode window through one MoE layer from C++, the way the reference engine calls its MoE half
// (src/engine.cu:933-978), through the C++ face over the C ABI (sfnx/kernels.hpp): quantize_q8_1, router_route,
// moe_gate_up, moe_down and the combine; then the same window through the fused decode.  Twice: with the shared
// expert as expert E of the stores, and as dense Q8_0 matrices through router_route's and moe_gate_up's shared-expert
// arguments (the reference's fused-shexp calls).  Prints "ok" when the two paths agree bit for bit; exit status 1
// otherwise.  Built by the package's build step; run by tests/test_gpu_cpp.py.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <vector>

#include "sfnx/kernels.hpp"

using namespace sfnx;

namespace {

void hk(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
template <typename T> T* dev(size_t n) {
    void* p = nullptr;
    hk(hipMalloc(&p, n * sizeof(T) + 256), "hipMalloc");
    hk(hipMemset(p, 0, n * sizeof(T) + 256), "hipMemset");
    return (T*) p;
}
// n_mat matrices of rows x cols, N(0, 0.02) from seed, quantized to `type` and packed into the planar store
void* synth_store(uint32_t type, int n_mat, int rows, int cols, uint64_t seed, uint64_t offset) {
    const size_t vals = (size_t) n_mat * rows * cols, bytes = (size_t) n_mat * rows * sfnx_row_bytes(type, cols);
    float* f = dev<float>(vals);
    uint8_t* g = dev<uint8_t>(bytes);
    uint8_t* p = dev<uint8_t>(bytes);
    ck(sfnx_synth_normal(f, vals, seed, offset, 0.02f, nullptr));
    ck(sfnx_quantize_weights(type, f, g, (int64_t) n_mat * rows, cols, nullptr));
    ck(sfnx_store_pack(type, g, p, n_mat, rows, cols, nullptr));
    hk(hipDeviceSynchronize(), "sync");
    hk(hipFree(f), "hipFree");
    hk(hipFree(g), "hipFree");
    return p;
}

bool run(bool dense_shared) {
    const MoeShape s{1024, 64, 6};
    const int ff = 512, T = 3, P = T * s.K, NP = P + T;
    const uint32_t type = T_Q4_K;
    const int E_store = dense_shared ? s.E : s.E + 1;
    const size_t gu_stride = 2 * (size_t) ff * sfnx_row_bytes(type, s.H), dn_stride = (size_t) s.H * sfnx_row_bytes(type, ff);
    float* W = dev<float>((size_t) (s.E + 1) * s.H);
    ck(sfnx_synth_normal(W, (size_t) (s.E + 1) * s.H, 11, 0, 0.02f, nullptr));
    const DW gu_e{synth_store(type, E_store, 2 * ff, s.H, 12, 0), type, s.H, 2 * ff};
    const DW dn_e{synth_store(type, E_store, s.H, ff, 13, 0), type, ff, s.H};
    const Q8S sh_gu{dense_shared ? synth_store(T_Q8_0, 1, 2 * ff, s.H, 12, (uint64_t) s.E * 2 * ff * s.H) : nullptr};
    const Q8S sh_dn{dense_shared ? synth_store(T_Q8_0, 1, s.H, ff, 13, (uint64_t) s.E * s.H * ff) : nullptr};
    float* x = dev<float>((size_t) T * s.H);
    ck(sfnx_synth_normal(x, (size_t) T * s.H, 14, 0, 1.0f, nullptr));
    // the unfused calls
    uint8_t* xq = dev<uint8_t>(q8_1_bytes(s.H) * T);
    float* logits = dev<float>((size_t) T * (s.E + 1));
    int* topi = dev<int>(P);
    float* topw = dev<float>(P);
    Job* jg = dev<Job>(P + 1);
    Job* jd = dev<Job>(P + 1);
    int* nj = dev<int>(2);
    float* gu = dev<float>((size_t) NP * 2 * ff);
    float* part = dev<float>((size_t) NP * s.H);
    float* y = dev<float>((size_t) T * s.H);
    uint8_t* hq = dev<uint8_t>(q8_1_bytes(ff) * T);
    quantize_q8_1(x, xq, s.H, T, nullptr);
    if (dense_shared) {
        router_route(s, W, x, logits, T, topi, topw, jg, jd, nj, nullptr, &sh_gu, 2 * ff, xq, gu + (size_t) P * 2 * ff);
        moe_gate_up(gu_e, gu_stride, jg, nj, P + 1, xq, gu, nullptr, T, &sh_dn, ff, gu + (size_t) P * 2 * ff,
                    part + (size_t) P * s.H, hq);
    } else {
        router_route(s, W, x, logits, T, topi, topw, jg, jd, nj, nullptr);
        moe_gate_up(gu_e, gu_stride, jg, nj, P + 1, xq, gu, nullptr, T);
    }
    moe_down(dn_e, dn_stride, jd, nj, P + 1, gu, part, nullptr, T);
    moe_combine(s, part, topw, topi, logits, y, T, nullptr);
    // the fused decode on a copy of x, norm off: x += y
    float* xf = dev<float>((size_t) T * s.H);
    hk(hipMemcpy(xf, x, (size_t) T * s.H * 4, hipMemcpyDeviceToDevice), "copy");
    const size_t wsb = sfnx_moe_decode_workspace(T, s.H, s.E, s.K, ff, nullptr);
    uint8_t* ws = dev<uint8_t>(wsb);
    const sfnx_moe_layer_w lw{W, gu_e.p, gu_stride, dn_e.p, dn_stride};
    if (dense_shared) {
        const sfnx_moe_shared_q8s shw{sh_gu.p, sh_dn.p};
        ck(sfnx_moe_decode_q8s(&lw, &shw, 1, type, type, s.H, s.E, s.K, ff, xf, T, 0, 1e-6f, ws, wsb, 0, nullptr));
    } else {
        ck(sfnx_moe_decode(&lw, 1, type, s.H, s.E, s.K, ff, 1, xf, T, 0, 1e-6f, ws, wsb, 0, nullptr));
    }
    hk(hipDeviceSynchronize(), "sync");
    std::vector<float> hx(T * s.H), hy(T * s.H), hf(T * s.H);
    hk(hipMemcpy(hx.data(), x, hx.size() * 4, hipMemcpyDeviceToHost), "copy");
    hk(hipMemcpy(hy.data(), y, hy.size() * 4, hipMemcpyDeviceToHost), "copy");
    hk(hipMemcpy(hf.data(), xf, hf.size() * 4, hipMemcpyDeviceToHost), "copy");
    size_t bad = 0;
    for (size_t i = 0; i < hx.size(); ++i) {
        const float want = hx[i] + hy[i];
        bad += std::memcmp(&want, &hf[i], 4) != 0;
    }
    std::printf("%s shared expert: %zu of %zu values differ\n", dense_shared ? "dense Q8_0" : "expert E", bad, hx.size());
    return bad == 0;
}

}  // namespace

int main() {
    try {
        const bool a = run(false), b = run(true);
        std::printf("%s\n", a && b ? "ok" : "MISMATCH");
        return a && b ? 0 : 1;
    } catch (const std::exception& e) {
        std::printf("error: %s\n", e.what());
        return 2;
    }
}
