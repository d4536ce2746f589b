"""CPU restatement of the expert cache's slot plan.  TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of
the library's sfnx_cache_plan, never by the sfnx_amd package.

cache_plan follows src/moe.cuh:22-71 (cache_plan, one warp): the window's jobs whose experts hold a slot mark it ref 2;
each other job, in job order, takes the first slot of the layer's pool that the CLOCK hand reaches with ref 0, looking
at 32 slots a step (the warp's lanes, slot (hand + lane) mod n), the ref-1 slots before the found one in that step
dropping to 0; a step without a ref-0 slot drops all its ref-1 slots and moves the hand 32 on.  The victim's old expert
goes back to its host copy.  Afterwards every job's slot is ref 1 and the hand is stored.  A miss that finds no victim
(every slot of the pool held by the window: two full turns of the hand see only ref 2) stays on its host copy, and so
do the misses after it; the state keeps the count in `left` (the library's status[0]; the reference's plan spins).

Pinned in tests/test_oracle_cache.py by: a case worked by hand (a pool of 5 slots, fewer than 32, where the 32-lane
steps alias slots), invariants over random windows (every job's expert in a slot, owner and slot_of inverse, the list
equal to the misses in job order, refs after the plan), and, for pools of 32 slots or more, equality with an
independently written one-slot-at-a-time second-chance CLOCK (the textbook algorithm, to which the 32-slot steps
reduce when no step sees a slot twice).
"""
from __future__ import annotations

SWEEP = 32


class PoolState:
    """one pool's part of the cache state (src/model.hpp:95-116): slot numbers s0 .. s0 + n - 1"""

    def __init__(self, n_layers: int, n_experts: int, n: int, s0: int = 0):
        self.E, self.n, self.s0 = n_experts, n, s0
        self.slot_of = [-1] * (n_layers * n_experts)
        self.owner = [-1] * (s0 + n)
        self.ref = [0] * (s0 + n)
        self.hand = s0
        self.left = 0

    def copy(self) -> "PoolState":
        c = PoolState.__new__(PoolState)
        c.E, c.n, c.s0 = self.E, self.n, self.s0
        c.slot_of, c.owner, c.ref, c.hand = list(self.slot_of), list(self.owner), list(self.ref), self.hand
        c.left = self.left
        return c


def cache_plan(st: PoolState, job_experts: list[int], layer: int) -> list[int]:
    """src/moe.cuh:22-71 for one layer whose pool is st; job_experts: each job's expert, in job order.  Returns the
    experts (layer * E + e) that took a slot, in job order; st.left receives the misses left on their host copies"""
    base, s0, n = layer * st.E, st.s0, st.n
    for e in job_experts:
        s = st.slot_of[base + e]
        if s >= 0:
            st.ref[s] = 2
    hand = st.hand - s0
    if hand < 0 or hand >= n:
        hand = 0
    taken = []
    left = 0
    failed = False
    for j0 in range(0, len(job_experts), SWEEP):
        group = job_experts[j0:j0 + SWEEP]
        misses = [j0 + i for i, e in enumerate(group) if st.slot_of[base + e] < 0]
        if failed:
            left += len(misses)
            continue
        for mi, j in enumerate(misses):
            g = base + job_experts[j]
            victim, steps = -1, 0
            while victim < 0:
                if steps > 2 * (n // SWEEP + 2):
                    failed = True
                    break
                steps += 1
                idx = [(hand + lane) % n for lane in range(SWEEP)]
                r = [st.ref[s0 + i] for i in idx]   # every lane reads before any writes
                f = next((lane for lane in range(SWEEP) if r[lane] == 0), SWEEP)
                for lane in range(f):
                    if r[lane] == 1:
                        st.ref[s0 + idx[lane]] = 0
                if f < SWEEP:
                    victim = (hand + f) % n
                hand = (hand + (f + 1 if f < SWEEP else SWEEP)) % n
            if failed:
                left += len(misses) - mi
                break
            vs = s0 + victim
            o = st.owner[vs]
            if o >= 0:
                st.slot_of[o] = -1
            st.owner[vs] = g
            st.slot_of[g] = vs
            st.ref[vs] = 2
            taken.append(g)
    for e in job_experts:
        if st.slot_of[base + e] >= 0:
            st.ref[st.slot_of[base + e]] = 1
    st.hand = s0 + hand
    st.left = left
    return taken
