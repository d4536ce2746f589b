// The expert cache's window plan (src/moe.cuh:22-71 cache_plan) as a device function of one wavefront, run by the
// plan kernel of its own (cache.hip) and by the last block of the decode router (route.hip), as the reference runs it.
#pragma once
#include "common.hpp"

namespace sfnx {

constexpr int EC_MAX_POOL = 32768;   // slots a pool may have: the plan keeps the pool's ref bytes in LDS
constexpr int EC_MAX_JOBS = 1024;    // jobs a plan takes: their slots are kept in LDS
constexpr int EC_SWEEP = 32;         // slots a CLOCK step looks at: the reference's warp

// The ordering a plan needs between its lanes' LDS accesses: a block barrier when the plan's wavefront is the whole
// workgroup, a wavefront fence and barrier when the other wavefronts of the block have left.
struct BlockSync {
    __device__ void operator()() const { __syncthreads(); }
};
struct WaveSync {
    __device__ void operator()() const {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
};

// One wavefront plans the slots of the window's nj jobs for `layer`.  Jobs whose experts are in a slot keep it (ref 2
// during the plan); each miss, in job order, takes the first slot the pool's CLOCK hand reaches with ref 0, EC_SWEEP
// slots a step, the ref-1 slots passed dropping to 0; the victim's expert goes back to its host copy.  A miss finds no
// victim only when every slot of the pool is held by the window (two full turns see only ref 2): it and the misses
// after it stay on their host copies, where their table entries already point, and are counted in status.  Every slot
// the window holds ends at ref 1.  list receives the count of experts that took a slot, then their ids.
template <typename Sync>
__device__ void plan_window(const sfnx_job* __restrict__ jobs, int nj, int layer, const sfnx_expert_cache& ec,
                            int* __restrict__ list, int lane, Sync sync) {
    __shared__ unsigned char ref[EC_MAX_POOL];
    __shared__ int jslot[EC_MAX_JOBS];   // each job's slot, pool-relative
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
    sync();
    for (int j = lane; j < nj; j += WAVE) {
        const int s = ec.slot_of[base + jobs[j].w];
        jslot[j] = s >= 0 ? s - s0 : -1;
        if (s >= 0) ref[s - s0] = 2;
    }
    sync();
    int hand = ec.hand[p] - s0, k = 0;
    if (hand < 0 || hand >= n) hand = 0;
    bool fail = false;
    int left = 0;
    const bool sweeper = lane < EC_SWEEP;
    // the misses, EC_SWEEP jobs at a time (found side by side), taken in job order
    for (int j0 = 0; j0 < nj; j0 += EC_SWEEP) {
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
            for (int step = 0; victim < 0; ++step) {
                if (step > 2 * (n / EC_SWEEP + 2)) {
                    fail = true;
                    break;
                }
                const int idx = (hand + lane) % n;
                const unsigned char r = sweeper ? ref[idx] : 255;
                const unsigned long long fr = __ballot(sweeper && r == 0);
                const int f = fr ? __ffsll(fr) - 1 : EC_SWEEP;
                if (sweeper && lane < f && r == 1) ref[idx] = 0;
                if (fr) victim = (hand + f) % n;
                hand = (hand + (fr ? f + 1 : EC_SWEEP)) % n;
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
            sync();
        }
    }
    sync();
    // the window's slots are used: ref 1 for the next plans, whether or not every miss found a slot (a ref 2 left
    // behind would make its slot unevictable)
    for (int j = lane; j < nj; j += WAVE)
        if (jslot[j] >= 0) ref[jslot[j]] = 1;
    sync();
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

// host checks of a cache and a layer before a plan or a copy is launched
inline void check_cache(const sfnx_expert_cache* ec) {
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
inline void check_layer(const sfnx_expert_cache* ec, int layer) {
    require(layer >= 0 && layer < ec->n_layers, "layer out of range");
    require(ec->pool_of[layer] >= 0 && ec->pool_of[layer] < ec->n_pools, "the layer's pool is out of range");
}

}  // namespace sfnx
