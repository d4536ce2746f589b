// A decode window through one MoE layer from C++, the way the reference engine calls its MoE half
// (src/engine.cu:933-978), through the C++ face over the C ABI (sfnx/kernels.hpp): quantize_q8_1, router_route,
// moe_gate_up, moe_down and the combine; then the same window through the fused decode.  Three times: with the shared
// expert as expert E of the stores, as dense Q8_0 matrices through router_route's and moe_gate_up's shared-expert
// arguments (the reference's fused-shexp calls), and the latter again through the overloads that keep the reference's
// argument lists exactly (src/kernels.hpp:276-305; N, NEXP, TOPK from set_model_shape).  Then a prompt chunk through
// the prompt path's calls under the reference's names (router_logits, pf_route, moe_gate_up_mma, swiglu_h16,
// moe_down_mma, the combine): equal bit for bit to the fused gate|up + SwiGLU form, and near the int8 BigJob form.
// Then windows through an ExpertCache (the routed experts in page-locked host memory, VRAM slots planned by
// router_route and filled by moe_cache, the expert calls reading the cache's tables through DW::ep), each equal bit
// for bit to the same window through the resident store.
// Prints "ok" when every check holds; exit status 1 otherwise.  Built by the package's build step; run by
// tests/test_gpu_cpp.py.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
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

// a dense Q8_0 matrix of rows x cols, N(0, 0.02) from seed, quantized and split on the host into the two planes the
// reference's loader fills (src/model.cpp:384-440 q8split: int8 values [rows][cols], f16 scale bits [rows][cols / 32]),
// each its own device allocation
Q8S synth_q8s(int rows, int cols, uint64_t seed, uint64_t offset) {
    const size_t vals = (size_t) rows * cols, nb = vals / 32;
    float* f = dev<float>(vals);
    uint8_t* g = dev<uint8_t>(nb * 34);
    ck(sfnx_synth_normal(f, vals, seed, offset, 0.02f, nullptr));
    ck(sfnx_quantize_weights(T_Q8_0, f, g, rows, cols, nullptr));
    std::vector<uint8_t> blocks(nb * 34);
    hk(hipMemcpy(blocks.data(), g, blocks.size(), hipMemcpyDeviceToHost), "copy");
    hk(hipFree(f), "hipFree");
    hk(hipFree(g), "hipFree");
    std::vector<int8_t> q(vals);
    std::vector<uint16_t> d(nb);
    for (size_t b = 0; b < nb; ++b) {
        std::memcpy(&d[b], &blocks[b * 34], 2);
        std::memcpy(&q[b * 32], &blocks[b * 34 + 2], 32);
    }
    Q8S m{dev<int8_t>(vals), dev<uint16_t>(nb)};
    hk(hipMemcpy(m.q, q.data(), vals, hipMemcpyHostToDevice), "copy");
    hk(hipMemcpy(m.d, d.data(), nb * 2, hipMemcpyHostToDevice), "copy");
    return m;
}

// mode 0: shared expert as expert E; 1: dense Q8_0 through the MoeShape overloads; 2: dense Q8_0 through the
// reference's exact argument lists
bool run(int mode) {
    const bool dense_shared = mode != 0;
    const MoeShape s{1024, 64, 6};
    const int ff = 512, T = 3, P = T * s.K, NP = P + T;
    const uint32_t type = T_Q4_K;
    const int E_store = dense_shared ? s.E : s.E + 1;
    const size_t gu_stride = 2 * (size_t) ff * sfnx_row_bytes(type, s.H), dn_stride = (size_t) s.H * sfnx_row_bytes(type, ff);
    float* W = dev<float>((size_t) (s.E + 1) * s.H);
    ck(sfnx_synth_normal(W, (size_t) (s.E + 1) * s.H, 11, 0, 0.02f, nullptr));
    const DW gu_e{synth_store(type, E_store, 2 * ff, s.H, 12, 0), type, s.H, 2 * ff};
    const DW dn_e{synth_store(type, E_store, s.H, ff, 13, 0), type, ff, s.H};
    const Q8S sh_gu = dense_shared ? synth_q8s(2 * ff, s.H, 12, (uint64_t) s.E * 2 * ff * s.H) : Q8S{nullptr, nullptr};
    const Q8S sh_dn = dense_shared ? synth_q8s(s.H, ff, 13, (uint64_t) s.E * s.H * ff) : Q8S{nullptr, nullptr};
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
    if (mode == 2) {   // src/engine.cu:952-971, word for word but for the buffers' names
        set_model_shape(s);
        router_route(W, x, logits, T, topi, topw, jg, jd, nj, nullptr, nullptr, -1, nullptr, &sh_gu, 2 * ff, xq,
                     gu + (size_t) P * 2 * ff);
        moe_gate_up(gu_e, gu_stride, jg, nj, P, xq, gu, nullptr, &sh_dn, ff, gu + (size_t) P * 2 * ff, part + (size_t) P * s.H);
        moe_down(dn_e, dn_stride, jd, nj, P, gu, part, nullptr);
    } else if (dense_shared) {
        router_route(s, W, x, logits, T, topi, topw, jg, jd, nj, nullptr, &sh_gu, 2 * ff, xq, gu + (size_t) P * 2 * ff);
        moe_gate_up(gu_e, gu_stride, jg, nj, P + 1, xq, gu, nullptr, T, &sh_dn, ff, gu + (size_t) P * 2 * ff,
                    part + (size_t) P * s.H, hq);
        moe_down(dn_e, dn_stride, jd, nj, P + 1, gu, part, nullptr, T);
    } else {
        router_route(s, W, x, logits, T, topi, topw, jg, jd, nj, nullptr);
        moe_gate_up(gu_e, gu_stride, jg, nj, P + 1, xq, gu, nullptr, T);
        moe_down(dn_e, dn_stride, jd, nj, P + 1, gu, part, nullptr, T);
    }
    moe_combine(s, part, topw, topi, logits, y, T, nullptr);
    // the fused decode on a copy of x, norm off: x += y
    float* xf = dev<float>((size_t) T * s.H);
    hk(hipMemcpy(xf, x, (size_t) T * s.H * 4, hipMemcpyDeviceToDevice), "copy");
    const size_t wsb = sfnx_moe_decode_workspace(T, s.H, s.E, s.K, ff, nullptr);
    uint8_t* ws = dev<uint8_t>(wsb);
    const sfnx_moe_layer_w lw{W, gu_e.p, gu_stride, dn_e.p, dn_stride};
    if (dense_shared) {
        const sfnx_moe_shared_q8s shw{sh_gu, sh_dn};
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
    static const char* names[3] = {"expert E", "dense Q8_0", "dense Q8_0, the reference's argument lists"};
    std::printf("%s shared expert: %zu of %zu values differ\n", names[mode], bad, hx.size());
    return bad == 0;
}

std::vector<float> host(const float* d, size_t n) {
    std::vector<float> h(n);
    hk(hipMemcpy(h.data(), d, n * 4, hipMemcpyDeviceToHost), "copy");
    return h;
}

// A prompt chunk of C tokens (src/prefill.cu:1145-1180) through the reference-named prompt calls
bool run_prompt() {
    const MoeShape s{1024, 64, 6};
    const int ff = 512, C = 96, P = C * s.K, NP = P + C;
    const uint32_t type = T_Q4_K;
    const size_t gu_stride = 2 * (size_t) ff * sfnx_row_bytes(type, s.H), dn_stride = (size_t) s.H * sfnx_row_bytes(type, ff);
    float* W = dev<float>((size_t) (s.E + 1) * s.H);
    ck(sfnx_synth_normal(W, (size_t) (s.E + 1) * s.H, 21, 0, 0.02f, nullptr));
    const DW gu_e{synth_store(type, s.E + 1, 2 * ff, s.H, 22, 0), type, s.H, 2 * ff};
    const DW dn_e{synth_store(type, s.E + 1, s.H, ff, 23, 0), type, ff, s.H};
    float* x = dev<float>((size_t) C * s.H);
    ck(sfnx_synth_normal(x, (size_t) C * s.H, 24, 0, 1.0f, nullptr));
    const int cap = P / 64 + s.E + (C + 63) / 64 + 1;
    float* logits = dev<float>((size_t) C * (s.E + 1));
    int* topi = dev<int>(P);
    float* topw = dev<float>(P);
    int* cnt = dev<int>(s.E);
    int* jbase = dev<int>(s.E);
    BigJob* jg = dev<BigJob>(cap);
    BigJob* jd = dev<BigJob>(cap);
    int* nj = dev<int>(2);
    uint16_t* xh = dev<uint16_t>((size_t) C * s.H);
    float* gu = dev<float>((size_t) NP * 2 * ff);
    uint16_t* h16 = dev<uint16_t>((size_t) NP * ff);
    uint16_t* h16f = dev<uint16_t>((size_t) NP * ff);
    float* part = dev<float>((size_t) NP * s.H);
    float* y1 = dev<float>((size_t) C * s.H);
    float* y2 = dev<float>((size_t) C * s.H);
    float* y3 = dev<float>((size_t) C * s.H);
    uint8_t* xq = dev<uint8_t>(q8_1_bytes(s.H) * C);
    router_logits(W, x, logits, C, s.H, s.E + 1, nullptr);
    pf_route(s, logits, C, topi, topw, cnt, jbase, jg, jd, nj, nullptr);
    ck(sfnx_to_f16(x, xh, (size_t) C * s.H, nullptr));
    // src/prefill.cu:1167-1171 as the reference writes it
    moe_gate_up_mma(gu_e, gu_stride, jg, nj, cap, xh, gu, nullptr);
    swiglu_h16(gu, ff, NP, h16, nullptr);
    moe_down_mma(dn_e, dn_stride, jd, nj, cap, h16, part, nullptr);
    moe_combine(s, part, topw, topi, logits, y1, C, nullptr);
    // the fused gate|up + SwiGLU form
    ck(sfnx_moe_gate_up_swiglu_mma(gu_e.p, gu_stride, type, s.H, ff, jg, nj, cap, xh, h16f, nullptr));
    moe_down_mma(dn_e, dn_stride, jd, nj, cap, h16f, part, nullptr);
    moe_combine(s, part, topw, topi, logits, y2, C, nullptr);
    // the int8 BigJob form (FNX_PF_MOE_Q8)
    quantize_q8_1(x, xq, s.H, C, nullptr);
    moe_gate_up_big(gu_e, gu_stride, jg, nj, cap, xq, gu, nullptr);
    moe_down_big(dn_e, dn_stride, jd, nj, cap, gu, part, nullptr);
    moe_combine(s, part, topw, topi, logits, y3, C, nullptr);
    hk(hipDeviceSynchronize(), "sync");
    const size_t n = (size_t) C * s.H;
    const std::vector<float> a = host(y1, n), b = host(y2, n), c = host(y3, n);
    size_t bad = 0;
    double dmax = 0, amax = 0;
    for (size_t i = 0; i < n; ++i) {
        bad += std::memcmp(&a[i], &b[i], 4) != 0;
        dmax = std::max(dmax, (double) std::fabs(a[i] - c[i]));
        amax = std::max(amax, (double) std::fabs(c[i]));
    }
    const double rel = dmax / amax;
    std::printf("prompt chunk of %d: fused gate|up+SwiGLU differs in %zu of %zu values; f16 vs int8 path max rel %.3g\n", C,
                bad, n, rel);
    return bad == 0 && rel < 5e-2;
}

// Windows through the expert cache, the engine's sequence (src/engine.cu:947-971) with `ec` live: router_route plans
// the window's slots, moe_cache copies the planned experts in, moe_gate_up / moe_down read the tables (DW::ep)
bool run_cached() {
    const MoeShape s{1024, 64, 6};
    const int ff = 512, T = 3, P = T * s.K, NP = P + T, n_slots = 24;
    const uint32_t type = T_Q4_K;
    set_model_shape(s);
    const size_t gu_stride = 2 * (size_t) ff * sfnx_row_bytes(type, s.H), dn_stride = (size_t) s.H * sfnx_row_bytes(type, ff);
    float* W = dev<float>((size_t) (s.E + 1) * s.H);
    ck(sfnx_synth_normal(W, (size_t) (s.E + 1) * s.H, 31, 0, 0.02f, nullptr));
    const DW gu_e{synth_store(type, s.E, 2 * ff, s.H, 32, 0), type, s.H, 2 * ff};
    const DW dn_e{synth_store(type, s.E, s.H, ff, 33, 0), type, ff, s.H};
    const Q8S sh_gu = synth_q8s(2 * ff, s.H, 32, (uint64_t) s.E * 2 * ff * s.H);
    const Q8S sh_dn = synth_q8s(s.H, ff, 33, (uint64_t) s.E * s.H * ff);
    // the cache: host copies of every expert, one pool of n_slots empty slots, the tables at the host copies
    void *hg = nullptr, *hgd = nullptr, *hd = nullptr, *hdd = nullptr;
    ck(sfnx_host_alloc(gu_stride * s.E, &hg, &hgd));
    ck(sfnx_host_alloc(dn_stride * s.E, &hd, &hdd));
    hk(hipMemcpy(hg, gu_e.p, gu_stride * s.E, hipMemcpyDeviceToHost), "copy");
    hk(hipMemcpy(hd, dn_e.p, dn_stride * s.E, hipMemcpyDeviceToHost), "copy");
    std::vector<const void*> tg(s.E), td(s.E);
    for (int e = 0; e < s.E; ++e) {
        tg[e] = (const char*) hgd + (size_t) e * gu_stride;
        td[e] = (const char*) hdd + (size_t) e * dn_stride;
    }
    ExpertCache ec{};
    ec.n_slots = n_slots;
    ec.n_pools = 1;
    ec.n_layers = 1;
    ec.n_experts = s.E;
    ec.pool_of[0] = 0;
    ec.s0[0] = 0;
    ec.n[0] = n_slots;
    ec.slot_bytes[0] = gu_stride + dn_stride;
    ec.dn_off[0] = gu_stride;
    ec.pool[0] = dev<uint8_t>((gu_stride + dn_stride) * n_slots);
    const void** ep_gu = dev<const void*>(s.E);
    const void** ep_dn = dev<const void*>(s.E);
    const void** host_gu = dev<const void*>(s.E);
    const void** host_dn = dev<const void*>(s.E);
    for (const void** t : {ep_gu, host_gu}) hk(hipMemcpy(t, tg.data(), s.E * sizeof(void*), hipMemcpyHostToDevice), "copy");
    for (const void** t : {ep_dn, host_dn}) hk(hipMemcpy(t, td.data(), s.E * sizeof(void*), hipMemcpyHostToDevice), "copy");
    ec.ep_gu = ep_gu;
    ec.ep_dn = ep_dn;
    ec.host_gu = host_gu;
    ec.host_dn = host_dn;
    ec.slot_of = dev<int>(s.E);
    ec.owner = dev<int>(n_slots);
    hk(hipMemset(ec.slot_of, 0xff, s.E * sizeof(int)), "memset");
    hk(hipMemset(ec.owner, 0xff, n_slots * sizeof(int)), "memset");
    ec.ref = dev<unsigned char>(n_slots);
    ec.hand = dev<int>(SFNX_EC_POOLS);
    DW gu_c = gu_e, dn_c = dn_e;   // the layer's experts through the cache's tables
    gu_c.p = dn_c.p = nullptr;
    gu_c.ep = (const char* const*) ep_gu;
    dn_c.ep = (const char* const*) ep_dn;
    uint8_t* xq = dev<uint8_t>(q8_1_bytes(s.H) * T);
    float* logits = dev<float>((size_t) T * (s.E + 1));
    int* topi = dev<int>(P);
    float* topw = dev<float>(P);
    Job* jg = dev<Job>(P + 1);
    Job* jd = dev<Job>(P + 1);
    int* nj = dev<int>(2);
    int* list = dev<int>(P + 2);
    float* gu = dev<float>((size_t) NP * 2 * ff);
    float* part = dev<float>((size_t) NP * s.H);
    float* y0 = dev<float>((size_t) T * s.H);
    float* y1 = dev<float>((size_t) T * s.H);
    float* x = dev<float>((size_t) T * s.H);
    size_t bad = 0;
    int planned = 0;
    for (int w = 0; w < 4; ++w) {
        ck(sfnx_synth_normal(x, (size_t) T * s.H, 40 + w, 0, 1.0f, nullptr));
        quantize_q8_1(x, xq, s.H, T, nullptr);
        for (int cached = 0; cached < 2; ++cached) {
            float* y = cached ? y1 : y0;
            router_route(W, x, logits, T, topi, topw, jg, jd, nj, nullptr, cached ? &ec : nullptr, 0, list, &sh_gu, 2 * ff,
                         xq, gu + (size_t) P * 2 * ff);
            if (cached) moe_cache(0, gu_stride, dn_stride, ec, list, nullptr);
            moe_gate_up(cached ? gu_c : gu_e, gu_stride, jg, nj, P, xq, gu, nullptr, &sh_dn, ff, gu + (size_t) P * 2 * ff,
                        part + (size_t) P * s.H);
            moe_down(cached ? dn_c : dn_e, dn_stride, jd, nj, P, gu, part, nullptr);
            moe_combine(s, part, topw, topi, logits, y, T, nullptr);
        }
        hk(hipDeviceSynchronize(), "sync");
        const std::vector<float> a = host(y0, (size_t) T * s.H), b = host(y1, (size_t) T * s.H);
        for (size_t i = 0; i < a.size(); ++i) bad += std::memcmp(&a[i], &b[i], 4) != 0;
        int n = 0;
        hk(hipMemcpy(&n, list, sizeof(int), hipMemcpyDeviceToHost), "copy");
        if (n < 0) ++bad;
        planned += n;
    }
    ck(sfnx_host_free(hg));
    ck(sfnx_host_free(hd));
    std::printf("expert cache (%d slots for %d experts): 4 windows, %d experts copied in, %zu values differ from the resident store\n",
                n_slots, s.E, planned, bad);
    return bad == 0 && planned > 0;
}

}  // namespace

int main() {
    try {
        const bool a = run(0), b = run(1), c = run(2), d = run_prompt(), e = run_cached();
        const bool ok = a && b && c && d && e;
        std::printf("%s\n", ok ? "ok" : "MISMATCH");
        return ok ? 0 : 1;
    } catch (const std::exception& e) {
        std::printf("error: %s\n", e.what());
        return 2;
    }
}
