// The expert cache for routed experts kept in host memory (src/model.hpp:95-116 ExpertCache, src/moe.cuh:19-71
// cache_plan, src/kernels.cu:1636-1668 k_cache_plan / k_cache_copy / moe_cache).  Every expert has a copy in
// page-locked host memory the GPU can read; VRAM holds slots, one pool of them per expert size, and the tables
// ep_gu / ep_dn say where each expert is now.  Before a decode window's expert kernels, one wavefront plans the
// window's slots (CLOCK over the layer's pool) and a copy kernel brings the planned experts in from their host copies;
// the expert kernels then read the layer's table rows as their stores (stride 0).
#include "common.hpp"

namespace sfnx {
namespace {

constexpr int EC_MAX_POOL = 32768;   // slots a pool may have: the plan keeps the pool's ref bytes in LDS
constexpr int EC_MAX_JOBS = 1024;    // jobs a plan takes: their slots are kept in LDS
constexpr int SWEEP = 32;            // slots a CLOCK step looks at: the reference's warp

__global__ void __launch_bounds__(WAVE) k_cache_plan(const sfnx_job* __restrict__ jobs, const int* __restrict__ njobs,
                                                     int layer, sfnx_expert_cache ec, int* __restrict__ list) {
    __shared__ unsigned char ref[EC_MAX_POOL];
    __shared__ int jslot[EC_MAX_JOBS];   // each job's slot, pool-relative
    const int lane = threadIdx.x, nj = *njobs;
    const int base = layer * ec.n_experts, p = ec.pool_of[layer], s0 = ec.s0[p], n = ec.n[p];
    if (nj < 0 || nj > EC_MAX_JOBS) {   // a count past what a plan takes: nothing planned, every miss from its host copy
        if (lane == 0) {
            list[0] = 0;
            if (ec.status) {
                ec.status[0] = max(nj, 0);
                ec.status[1] += max(nj, 0);
            }
        }
        return;
    }
    for (int i = lane; i < n; i += WAVE) ref[i] = ec.ref[s0 + i];
    __syncthreads();
    // the jobs whose experts are in a slot keep it: ref 2, not to be taken by this plan
    for (int j = lane; j < nj; j += WAVE) {
        const int s = ec.slot_of[base + jobs[j].w];
        jslot[j] = s >= 0 ? s - s0 : -1;
        if (s >= 0) ref[s - s0] = 2;
    }
    __syncthreads();
    int hand = ec.hand[p] - s0, k = 0;
    if (hand < 0 || hand >= n) hand = 0;
    // A miss finds no victim only when every slot of the pool is held by this window (ref 2).  It then stays on its
    // host copy, where its table entries already point (the expert kernels read it there, over the bus), and so do
    // the misses after it; the experts planned before it keep their slots and are copied in.
    bool fail = false;
    int left = 0;
    const bool sweeper = lane < SWEEP;
    // the misses, SWEEP jobs at a time (found side by side), taken in job order
    for (int j0 = 0; j0 < nj; j0 += SWEEP) {
        unsigned long long miss = __ballot(sweeper && j0 + lane < nj && jslot[j0 + lane] < 0);
        if (fail) {
            left += __popcll(miss);
            continue;
        }
        while (miss) {
            const int jm = j0 + __ffsll(miss) - 1;
            miss &= miss - 1;
            const int g = base + jobs[jm].w;
            int victim = -1;
            // CLOCK: the first slot from the hand with ref 0; the ref-1 slots passed before it drop to 0.  A pool whose
            // slots all hold ref 2 has no victim: two full turns end the search
            for (int step = 0; victim < 0; ++step) {
                if (step > 2 * (n / SWEEP + 2)) {
                    fail = true;
                    break;
                }
                const int idx = (hand + lane) % n;
                const unsigned char r = sweeper ? ref[idx] : 255;
                const unsigned long long fr = __ballot(sweeper && r == 0);
                const int f = fr ? __ffsll(fr) - 1 : SWEEP;
                if (sweeper && lane < f && r == 1) ref[idx] = 0;
                if (fr) victim = (hand + f) % n;
                hand = (hand + (fr ? f + 1 : SWEEP)) % n;
            }
            if (fail) {
                left += 1 + __popcll(miss);   // this miss and the rest of its group
                break;
            }
            if (lane == 0) {
                const int vs = s0 + victim, o = ec.owner[vs];
                if (o >= 0) {   // the victim's expert back to its host copy
                    ec.slot_of[o] = -1;
                    ec.ep_gu[o] = ec.host_gu[o];
                    ec.ep_dn[o] = ec.host_dn[o];
                }
                ec.owner[vs] = g;
                ec.slot_of[g] = vs;
                const char* at = static_cast<const char*>(ec.pool[p]) + (size_t) victim * ec.slot_bytes[p];
                ec.ep_gu[g] = at;
                ec.ep_dn[g] = at + ec.dn_off[p];
                list[1 + k] = g;
                ref[victim] = 2;
                jslot[jm] = victim;
            }
            ++k;
            __syncthreads();
        }
    }
    __syncthreads();
    // the window's slots are used: ref 1 for the next plans, whether or not every miss found a slot (a ref 2 left
    // behind would make its slot unevictable)
    for (int j = lane; j < nj; j += WAVE)
        if (jslot[j] >= 0) ref[jslot[j]] = 1;
    __syncthreads();
    for (int i = lane; i < n; i += WAVE) ec.ref[s0 + i] = ref[i];
    if (lane == 0) {
        ec.hand[p] = s0 + hand;
        list[0] = k;
        if (ec.status) {
            ec.status[0] = left;
            ec.status[1] += left;
        }
    }
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

void check_cache(const sfnx_expert_cache* ec) {
    require(ec != nullptr, "null expert cache");
    require(ec->n_pools >= 1 && ec->n_pools <= SFNX_EC_POOLS, "n_pools out of range");
    require(ec->n_layers >= 1 && ec->n_layers <= SFNX_EC_LAYERS && ec->n_experts >= 1, "table shape out of range");
    require(ec->ep_gu && ec->ep_dn && ec->host_gu && ec->host_dn && ec->slot_of && ec->owner && ec->ref && ec->hand,
            "null table in the expert cache");
    for (int p = 0; p < ec->n_pools; ++p) {
        require(ec->pool[p] != nullptr && ec->n[p] >= 1 && ec->n[p] <= EC_MAX_POOL && ec->s0[p] >= 0 &&
                    ec->s0[p] + ec->n[p] <= ec->n_slots, "pool slots out of range");
        require(ec->slot_bytes[p] % 16 == 0 && ec->dn_off[p] % 16 == 0 && ec->dn_off[p] < ec->slot_bytes[p],
                "pool slot sizes must be multiples of 16 with down after gate|up");
    }
}
void check_layer(const sfnx_expert_cache* ec, int layer) {
    require(layer >= 0 && layer < ec->n_layers, "layer out of range");
    require(ec->pool_of[layer] >= 0 && ec->pool_of[layer] < ec->n_pools, "the layer's pool is out of range");
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
