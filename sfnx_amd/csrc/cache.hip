// The expert cache for routed experts kept in host memory (src/model.hpp:95-116 ExpertCache, src/moe.cuh:19-71
// cache_plan, src/kernels.cu:1636-1668 k_cache_plan / k_cache_copy / moe_cache).  Every expert has a copy in
// page-locked host memory the GPU can read; VRAM holds slots, one pool of them per expert size, and the tables
// ep_gu / ep_dn say where each expert is now.  Before a decode window's expert kernels, one wavefront plans the
// window's slots (CLOCK over the layer's pool) and a copy kernel brings the planned experts in from their host copies;
// the expert kernels then read the layer's table rows as their stores (stride 0).
#include "cache.hpp"

namespace sfnx {
namespace {

__global__ void __launch_bounds__(WAVE) k_cache_plan(const sfnx_job* __restrict__ jobs, const int* __restrict__ njobs,
                                                     int layer, sfnx_expert_cache ec, int* __restrict__ list) {
    plan_window(jobs, *njobs, layer, ec, list, threadIdx.x, BlockSync{});
}

// the listed experts' matrices (gu_bytes and dn_bytes each, multiples of 16) from their host copies into their slots
// of pool p, 16 bytes a lane
__global__ void __launch_bounds__(256) k_cache_copy(sfnx_expert_cache ec, int p, const int* __restrict__ list,
                                                    size_t gu_bytes, size_t dn_bytes) {
    const int n = list[0];
    const size_t ug = gu_bytes / 16, per = ug + dn_bytes / 16;
    for (size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x; i < (size_t) max(n, 0) * per; i += (size_t) gridDim.x * blockDim.x) {
        const int k = (int) (i / per), g = list[1 + k];
        const size_t o = i % per;
        char* at = static_cast<char*>(ec.pool[p]) + (size_t) (ec.slot_of[g] - ec.s0[p]) * ec.slot_bytes[p];
        // the host copies' table entries read as global-memory pointers (loads through them global, not flat)
        const auto* hg = reinterpret_cast<const global_u8_ptr*>(ec.host_gu);
        const auto* hd = reinterpret_cast<const global_u8_ptr*>(ec.host_dn);
        if (o < ug) reinterpret_cast<uint4*>(at)[o] = reinterpret_cast<const uint4*>((const uint8_t*) hg[g])[o];
        else reinterpret_cast<uint4*>(at + ec.dn_off[p])[o - ug] = reinterpret_cast<const uint4*>((const uint8_t*) hd[g])[o - ug];
    }
}

void cache_plan(const sfnx_job* jobs, const int* njobs, int layer, const sfnx_expert_cache* ec, int* list, hipStream_t s) {
    k_cache_plan<<<1, WAVE, 0, s>>>(jobs, njobs, layer, *ec, list);
}
void cache_copy(const sfnx_expert_cache* ec, int p, const int* list, hipStream_t s) {
    k_cache_copy<<<640, 256, 0, s>>>(*ec, p, list, ec->dn_off[p], ec->slot_bytes[p] - ec->dn_off[p]);
}

}  // namespace
}  // namespace sfnx

using namespace sfnx;

extern "C" int sfnx_host_alloc(size_t bytes, void** host, void** dev) {
    return guarded_host("sfnx_host_alloc", [&] {
        require(host != nullptr && dev != nullptr && bytes > 0, "null output or zero bytes");
        void* h = nullptr;
        check(hipHostMalloc(&h, bytes, hipHostMallocMapped), "hipHostMalloc");
        void* d = nullptr;
        const hipError_t e = hipHostGetDevicePointer(&d, h, 0);
        if (e != hipSuccess) {
            (void) hipHostFree(h);
            check(e, "hipHostGetDevicePointer");
        }
        *host = h;
        *dev = d;
    });
}

extern "C" int sfnx_host_free(void* host) {
    return guarded_host("sfnx_host_free", [&] { check(hipHostFree(host), "hipHostFree"); });
}

extern "C" int sfnx_cache_plan(const sfnx_job* jobs, const int* njobs, int layer, const sfnx_expert_cache* ec, int* list,
                               void* st) {
    return guarded("sfnx_cache_plan", [&] {
        require(jobs != nullptr && njobs != nullptr && list != nullptr, "null pointer");
        check_cache(ec);
        check_layer(ec, layer);
        cache_plan(jobs, njobs, layer, ec, list, stream_of(st));
    });
}

extern "C" int sfnx_cache_copy(const sfnx_expert_cache* ec, int p, const int* list, void* st) {
    return guarded("sfnx_cache_copy", [&] {
        require(list != nullptr, "null list");
        check_cache(ec);
        require(p >= 0 && p < ec->n_pools, "pool out of range");
        cache_copy(ec, p, list, stream_of(st));
    });
}

extern "C" int sfnx_moe_cache(int layer, size_t gu_stride, size_t dn_stride, const sfnx_expert_cache* ec, int* list,
                              const sfnx_job* jobs, const int* njobs, void* st) {
    return guarded("sfnx_moe_cache", [&] {
        require(list != nullptr, "null list");
        check_cache(ec);
        check_layer(ec, layer);
        const int p = ec->pool_of[layer];
        require(gu_stride == ec->dn_off[p] && ec->dn_off[p] + dn_stride == ec->slot_bytes[p],
                "the layer's experts are not its pool's size");
        hipStream_t s = stream_of(st);
        if (jobs) {
            require(njobs != nullptr, "null njobs");
            cache_plan(jobs, njobs, layer, ec, list, s);
        }
        cache_copy(ec, p, list, s);
    });
}
