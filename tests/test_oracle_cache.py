"""The expert cache's slot plan restated on the CPU (oracle/cache.py, src/moe.cuh:22-71), pinned: a case worked by hand
on a pool smaller than the 32-lane sweep, invariants over random windows, and equality with an independently written
one-slot-at-a-time second-chance CLOCK for pools of 32 slots or more."""
import random

import pytest

from oracle.cache import PoolState, cache_plan


def test_hand_worked_pool_of_five():
    st = PoolState(n_layers=1, n_experts=10, n=5)
    assert cache_plan(st, [3, 7], 0) == [3, 7]
    assert (st.owner, st.ref, st.hand) == ([3, 7, -1, -1, -1], [1, 1, 0, 0, 0], 2)
    assert cache_plan(st, [7, 1, 4], 0) == [1, 4]            # 7 hits slot 1
    assert (st.owner, st.ref, st.hand) == ([3, 7, 1, 4, -1], [1, 1, 1, 1, 0], 4)
    assert cache_plan(st, [9, 3], 0) == [9]                  # the hand's slot 4 is free
    assert (st.owner, st.ref, st.hand) == ([3, 7, 1, 4, 9], [1, 1, 1, 1, 1], 0)
    # every slot ref 1: the first 32-lane step (slots 0..4 seen six times over) finds no ref 0, clears them all and
    # moves the hand 32 on, to slot 2; the next step takes slot 2 (expert 1 out), then slot 3 (expert 4 out).  A
    # one-slot-at-a-time CLOCK would have taken slot 0 here.
    assert cache_plan(st, [5, 6], 0) == [5, 6]
    assert (st.owner, st.ref, st.hand) == ([3, 7, 5, 6, 9], [0, 0, 1, 1, 0], 4)
    assert st.slot_of[1] == -1 and st.slot_of[4] == -1 and st.slot_of[5] == 2 and st.slot_of[6] == 3


def test_no_victim_leaves_the_rest_on_host():
    """three misses, two slots: the first two take the slots, the third finds every slot held by the window (five
    32-lane steps, the hand back at slot 0) and stays on its host copy; the window's slots end at ref 1, so the next
    window evicts as usual"""
    st = PoolState(n_layers=1, n_experts=10, n=2)
    assert cache_plan(st, [0, 1, 2], 0) == [0, 1]
    assert (st.owner, st.ref, st.hand, st.left) == ([0, 1], [1, 1], 0, 1)
    assert st.slot_of[2] == -1
    # every slot ref 1: the first step clears both and moves 32 on (slot 0); the second takes slot 0 (expert 0 out)
    assert cache_plan(st, [2], 0) == [2]
    assert (st.owner, st.ref, st.hand, st.left) == ([2, 1], [1, 0], 1, 0)
    assert st.slot_of[0] == -1
    # misses past the failing one in a later sweep group count too
    st = PoolState(n_layers=1, n_experts=80, n=1)
    assert cache_plan(st, list(range(40)), 0) == [0]
    assert st.left == 39 and st.ref == [1]


def clock_sequential(st: PoolState, jobs, layer):
    """second-chance CLOCK one slot at a time: ref 2 slots (this window's hits and takes) are passed, ref 1 ones drop
    to 0 as the hand passes, the first ref 0 one is taken"""
    base, s0, n = layer * st.E, st.s0, st.n
    for e in jobs:
        if st.slot_of[base + e] >= 0:
            st.ref[st.slot_of[base + e]] = 2
    misses = [e for e in jobs if st.slot_of[base + e] < 0]
    hand = st.hand - s0 if 0 <= st.hand - s0 < n else 0
    taken = []
    for e in misses:
        for _ in range(3 * n + 1):
            s = s0 + hand
            hand = (hand + 1) % n
            if st.ref[s] == 0:
                break
            if st.ref[s] == 1:
                st.ref[s] = 0
        else:
            return None
        if st.owner[s] >= 0:
            st.slot_of[st.owner[s]] = -1
        st.owner[s], st.slot_of[base + e], st.ref[s] = base + e, s, 2
        taken.append(base + e)
    for e in jobs:
        st.ref[st.slot_of[base + e]] = 1
    st.hand = s0 + hand
    return taken


def check_invariants(st: PoolState, jobs, layer, taken, before):
    base = layer * st.E
    for e in jobs:
        s = st.slot_of[base + e]
        assert st.s0 <= s < st.s0 + st.n and st.owner[s] == base + e and st.ref[s] == 1
    for s in range(st.s0, st.s0 + st.n):
        if st.owner[s] >= 0:
            assert st.slot_of[st.owner[s]] == s
        assert st.ref[s] in (0, 1)
    assert taken == [base + e for e in jobs if before.slot_of[base + e] < 0]


@pytest.mark.parametrize("n, E, nl", [(5, 12, 1), (17, 40, 2), (32, 64, 2), (40, 100, 3), (96, 200, 2), (257, 600, 2)])
def test_random_windows_invariants_and_sequential_clock(n, E, nl):
    rng = random.Random(n * 1000 + E)
    st = PoolState(nl, E, n, s0=3)
    seq = st.copy()
    for w in range(200):
        layer = rng.randrange(nl)
        k = rng.randint(1, min(n, 12, E))
        hot = list(range(min(E, n + 8)))   # skewed: mostly a hot set a bit larger than the pool
        jobs = rng.sample(hot if rng.random() < 0.8 else range(E), k)
        before = st.copy()
        taken = cache_plan(st, jobs, layer)
        assert taken is not None
        check_invariants(st, jobs, layer, taken, before)
        if n >= 32:
            t2 = clock_sequential(seq, jobs, layer)
            assert t2 == taken and seq.owner == st.owner and seq.ref == st.ref and seq.hand == st.hand
