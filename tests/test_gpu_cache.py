"""The expert cache (src/moe.cuh:19-71, src/kernels.cu:1636-1668): routed experts in page-locked host memory, VRAM
slots planned per decode window by one wavefront (CLOCK), in the router launch's last block as the reference's
(src/moe.cuh:128-198) or as a launch of its own, and filled by the copy kernel.  Each window through the cached
layer gives the same bits as the resident layer, and the device's plan (slots, owners, refs, hand, list) equals the
CPU restatement's (oracle/cache.py) window after window, for a pool larger and one smaller than the 32-lane sweep."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from oracle.cache import PoolState, cache_plan
from sfnx_amd import moe
from tests.gpu_util import job_array, make_layer

pytestmark = pytest.mark.gpu


def bits(t):
    return t.detach().cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("plan_in_router", [True, False])
@pytest.mark.parametrize("n_slots", [40, 24])
def test_cached_decode_windows(n_slots, plan_in_router):
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    layers = [make_layer(shape, 90 + l)[0] for l in range(2)]
    cache = moe.ExpertCache(layers, n_slots)
    E1 = cache.n_experts
    st = PoolState(len(layers), E1, n_slots)
    lst = torch.zeros(1 + 16 * shape.K + 16, dtype=torch.int32, device="cuda")
    rng = np.random.default_rng(n_slots)
    try:
        for w in range(24):
            l = w % 2
            T = int(rng.integers(1, 4))
            x = torch.from_numpy(orc.synth(T * shape.H, 1000 + w, 1.0).reshape(T, shape.H)).cuda()
            b0, b1 = moe.DecodeBuffers(shape, T), moe.DecodeBuffers(shape, T)
            y0, y1 = torch.empty_like(x), torch.empty_like(x)
            moe.decode_layer(layers[l], x, y0, b0)
            moe.decode_layer_cached(cache, l, x, y1, b1, lst, plan_in_router)
            torch.cuda.synchronize()
            assert np.array_equal(bits(y0), bits(y1)), f"window {w}"
            assert int(b1.njobs[1]) == 0   # the router's block counter left at zero
            nj = int(b1.njobs[0])
            jobs = [int(v) for v in job_array(b1.jobs_gu)[:nj]["w"]]
            taken = cache_plan(st, jobs, l)
            assert taken is not None
            got = lst.cpu().numpy()
            assert got[0] == len(taken) and list(got[1:1 + len(taken)]) == taken, f"window {w}"
            assert cache.slot_of.cpu().tolist() == st.slot_of
            assert cache.owner.cpu().tolist() == st.owner
            assert cache.ref.cpu().tolist() == st.ref
            assert int(cache.hand[0]) == st.hand
            # the tables: each expert at its slot or its host copy
            epg, hg = cache.ep_gu.cpu().numpy(), cache.host_gu.cpu().numpy()
            base = cache.pool.data_ptr()
            for g, s in enumerate(st.slot_of):
                want = base + s * cache.slot_bytes if s >= 0 else hg[g]
                assert epg[g] == want
    finally:
        cache.close()


@pytest.mark.parametrize("plan_in_router", [True, False])
def test_pool_too_small_leaves_misses_on_host(plan_in_router):
    """a window of 3 rows (more distinct experts than the pool's 12 slots) through the cache: the first 12 misses take
    the slots and are copied in, the others stay on their host copies (status[0]); the layer through the tables still
    equals the resident layer bit for bit, every table entry points at a slot holding that expert's bytes or at the
    expert's host copy, no ref is left at 2, the state equals the CPU restatement's; and the next windows of one row
    (7 jobs), which fit, plan and run as usual"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    layers = [make_layer(shape, 95)[0]]
    cache = moe.ExpertCache(layers, 12)
    E1 = cache.n_experts
    st = PoolState(1, E1, 12)
    lst = torch.zeros(64, dtype=torch.int32, device="cuda")
    try:
        lefts = []
        for w, T in enumerate((3, 1, 1, 2)):
            x = torch.from_numpy(orc.synth(T * shape.H, 1100 + w, 1.0).reshape(T, shape.H)).cuda()
            b0, b1 = moe.DecodeBuffers(shape, T), moe.DecodeBuffers(shape, T)
            y0, y1 = torch.empty_like(x), torch.empty_like(x)
            moe.decode_layer(layers[0], x, y0, b0)
            moe.decode_layer_cached(cache, 0, x, y1, b1, lst, plan_in_router)
            torch.cuda.synchronize()
            assert np.array_equal(bits(y0), bits(y1)), f"window {w}"
            nj = int(b1.njobs[0])
            jobs = [int(v) for v in job_array(b1.jobs_gu)[:nj]["w"]]
            taken = cache_plan(st, jobs, 0)
            got = lst.cpu().numpy()
            assert got[0] == len(taken) and list(got[1:1 + len(taken)]) == taken
            assert cache.host_misses()[0] == st.left
            lefts.append(st.left)
            if w == 0:
                assert nj > 12 and st.left == nj - 12
            if T == 1:
                assert st.left == 0
            assert cache.slot_of.cpu().tolist() == st.slot_of
            assert cache.owner.cpu().tolist() == st.owner
            assert cache.ref.cpu().tolist() == st.ref and 2 not in st.ref
            assert int(cache.hand[0]) == st.hand
            epg, hg = cache.ep_gu.cpu().numpy(), cache.host_gu.cpu().numpy()
            pool = cache.pool.cpu().numpy()
            gu_host = layers[0].gu_w.cpu().numpy()
            for g, s in enumerate(st.slot_of):
                if s >= 0:
                    assert epg[g] == cache.pool.data_ptr() + s * cache.slot_bytes
                    sl = pool[s * cache.slot_bytes: s * cache.slot_bytes + cache.gu_bytes]
                    assert np.array_equal(sl, gu_host[g * cache.gu_bytes:(g + 1) * cache.gu_bytes])
                else:
                    assert epg[g] == hg[g]
        assert cache.host_misses()[1] == sum(lefts)
    finally:
        cache.close()


def test_moe_cache_refuses_a_layer_of_another_size():
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    layers = [make_layer(shape, 96)[0]]
    cache = moe.ExpertCache(layers, 8)
    lst = torch.zeros(64, dtype=torch.int32, device="cuda")
    try:
        with pytest.raises(RuntimeError, match="pool's size"):
            moe.check(moe.lib().sfnx_moe_cache(0, cache.gu_bytes + 16, cache.dn_bytes, moe.C.byref(cache.c), lst.data_ptr(),
                                               None, None, moe._st()))
    finally:
        cache.close()



@pytest.mark.parametrize("plan_in_router", [True, False])
def test_cached_full_windows(plan_in_router):
    """16-row windows (the most a window holds: up to 97 jobs, several 32-job sweep groups a plan) over two layers
    through a 90-slot pool: outputs equal the resident layers' bit for bit, the plan equals the restatement's"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    layers = [make_layer(shape, 120 + l)[0] for l in range(2)]
    cache = moe.ExpertCache(layers, 90)
    st = PoolState(len(layers), cache.n_experts, 90)
    lst = torch.zeros(1 + 16 * shape.K + 16, dtype=torch.int32, device="cuda")
    T = 16
    try:
        for w in range(6):
            l = w % 2
            x = torch.from_numpy(orc.synth(T * shape.H, 1200 + w, 1.0).reshape(T, shape.H)).cuda()
            b0, b1 = moe.DecodeBuffers(shape, T), moe.DecodeBuffers(shape, T)
            y0, y1 = torch.empty_like(x), torch.empty_like(x)
            moe.decode_layer(layers[l], x, y0, b0)
            moe.decode_layer_cached(cache, l, x, y1, b1, lst, plan_in_router)
            torch.cuda.synchronize()
            assert np.array_equal(bits(y0), bits(y1)), f"window {w}"
            nj = int(b1.njobs[0])
            assert nj > 32   # more than one sweep group
            jobs = [int(v) for v in job_array(b1.jobs_gu)[:nj]["w"]]
            taken = cache_plan(st, jobs, l)
            got = lst.cpu().numpy()
            assert got[0] == len(taken) and list(got[1:1 + len(taken)]) == taken, f"window {w}"
            assert cache.host_misses()[0] == st.left == 0
            assert cache.slot_of.cpu().tolist() == st.slot_of
            assert cache.owner.cpu().tolist() == st.owner
            assert cache.ref.cpu().tolist() == st.ref
            assert int(cache.hand[0]) == st.hand
    finally:
        cache.close()
