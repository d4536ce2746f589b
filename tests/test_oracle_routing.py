"""Pins the oracle's routing: router logits against float64 products, top-k against brute-force sorting on the tie
cases of the reference's own top-k test (tools/topk_test.cu:110-164, here at the router's 512 experts), and the job /
permutation builders against their defining properties (src/moe.cuh:164-198, src/prefill.cu:223-279,
tools/kbench.cu:77-95).
"""
import numpy as np
import pytest

E, K = 512, 10


def brute_topk(row, E, K):
    """the K largest of row[:E] by (value desc, index asc); NaN and -inf never taken"""
    cand = [(-float(row[i]), i) for i in range(E) if np.isfinite(row[i]) or row[i] == np.inf]
    cand.sort()
    idx = [i for _, i in cand[:K]] + [-1] * (K - min(K, len(cand)))
    return idx


def check_rows(orc, rows):
    logits = np.ascontiguousarray(rows, np.float32)
    topi, topw, missing = orc.topk(logits, E, K)
    for t in range(logits.shape[0]):
        want = brute_topk(logits[t], E, K)
        assert topi[t].tolist() == want, t
        sel = [i for i in want if i >= 0]
        if sel:
            v = logits[t, sel].astype(np.float64)
            with np.errstate(invalid="ignore"):   # a +inf top logit: exp(inf - inf) is NaN, as in the reference
                w = np.exp(v - v[0])
                w /= w.sum()
            assert np.allclose(topw[t, :len(sel)], w, rtol=2e-6, atol=1e-7, equal_nan=True)
        assert np.all(topw[t, len(sel):] == 0)
    return topi, topw, missing


def test_router_logits_against_float64(orc):
    H, L, T = 2048, 513, 5
    W = orc.synth(L * H, 21, 0.02).reshape(L, H)
    x = orc.synth(T * H, 22, 1.0).reshape(T, H)
    got = orc.router_logits(W, x)
    exact = x.astype(np.float64) @ W.astype(np.float64).T
    bound = H * 2.0 ** -23 * (np.abs(x).astype(np.float64) @ np.abs(W).astype(np.float64).T)
    assert np.all(np.abs(got - exact) <= bound)
    # a one-hot router row reads one activation exactly
    W1 = np.zeros((3, H), np.float32)
    W1[0, 7], W1[1, 2047], W1[2, 1000] = 1, 2, -0.5
    l1 = orc.router_logits(W1, x)
    assert np.array_equal(l1, np.stack([x[:, 7], 2 * x[:, 2047], -0.5 * x[:, 1000]], 1))


@pytest.mark.parametrize("H", [1024, 2048, 2560, 4096])
def test_router_logits_mm_against_float64(orc, H):
    """the prompt path's order (8 slices of fmaf chains, added in slice order): within the fp32 summation bound of the
    float64 product, exact on one-hot rows and on integer data (every partial sum exact)"""
    L, T = 67, 5
    W = orc.synth(L * H, 23, 0.02).reshape(L, H)
    x = orc.synth(T * H, 24, 1.0).reshape(T, H)
    got = orc.router_logits_mm(W, x)
    exact = x.astype(np.float64) @ W.astype(np.float64).T
    bound = (H / 8 + 8) * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(W).astype(np.float64).T)
    assert np.all(np.abs(got - exact) <= bound)
    W1 = np.zeros((3, H), np.float32)
    W1[0, 7], W1[1, H - 1], W1[2, H // 2 + 3] = 1, 2, -0.5
    assert np.array_equal(orc.router_logits_mm(W1, x), np.stack([x[:, 7], 2 * x[:, H - 1], -0.5 * x[:, H // 2 + 3]], 1))
    rng = np.random.default_rng(H)
    Wi = rng.integers(-8, 9, (L, H)).astype(np.float32)
    xi = rng.integers(-8, 9, (T, H)).astype(np.float32)
    assert np.array_equal(orc.router_logits_mm(Wi, xi), (xi.astype(np.int64) @ Wi.astype(np.int64).T).astype(np.float32))
    # a different order from the decode router's: the two agree within the bound, not bit for bit everywhere
    assert np.all(np.abs(orc.router_logits(W, x) - got) <= 2 * bound)


def test_topk_random_rows(orc):
    rng = np.random.default_rng(7)
    check_rows(orc, rng.normal(0, 3, (12, E + 1)))


def test_topk_all_equal_and_all_zero(orc):
    topi, _, _ = check_rows(orc, np.stack([np.full(E + 1, 1.5), np.zeros(E + 1)]))
    assert topi.tolist() == [list(range(K))] * 2


def test_topk_tied_at_threshold(orc):
    r = np.full(E + 1, -5.0)
    for k in range(4):
        r[(k * 79) % E] = 9 + k
    for k in range(60):
        r[(k * 104729 + 13) % E] = 2.0
    check_rows(orc, r[None])


def test_topk_ties_straddling_lane_blocks(orc):
    # ties around multiples of 64 (the wavefront's lane blocks) and 32
    r = np.full(E + 1, -2.0)
    for c in range(1, 8):
        for d in range(-3, 3):
            r[64 * c + d] = 1.0
    check_rows(orc, r[None])


def test_topk_nan_inf_and_too_few(orc):
    r = np.full(E + 1, np.nan)
    r[[5, 400, 17]] = [1.0, 3.0, 1.0]
    r[[8, 9]] = -np.inf
    r[E] = 100.0  # the shared gate's logit is never a candidate
    topi, topw, missing = check_rows(orc, r[None])
    assert topi[0].tolist()[:3] == [400, 5, 17] and missing == K - 3
    r2 = np.full(E + 1, -1.0)
    r2[300] = np.inf
    check_rows(orc, r2[None])


def test_jobs_decode_properties(orc):
    rng = np.random.default_rng(8)
    for T in (1, 2, 3, 11, 16):
        topi = np.stack([rng.choice(E if T < 8 else 40, K, replace=False) for _ in range(T)]).astype(np.int32)
        for shared in (False, True):
            gu, dn = orc.jobs_decode(topi, K, E, shared)
            flat = topi.reshape(-1)
            first = []
            for p, e in enumerate(flat):
                if e not in first:
                    first.append(int(e))
            routed = gu[: len(first)]
            assert routed["w"].tolist() == first and dn["w"].tolist()[: len(first)] == first
            seen = []
            for j, job in enumerate(routed):
                pairs = job["out"][: job["n"]].tolist()
                assert pairs == sorted(pairs) and all(flat[p] == job["w"] for p in pairs)
                assert job["y"][: job["n"]].tolist() == [p // K for p in pairs]
                assert dn[j]["y"][: job["n"]].tolist() == pairs and dn[j]["out"][: job["n"]].tolist() == pairs
                seen += pairs
            assert sorted(seen) == list(range(T * K))
            assert len(gu) == len(first) + shared
            if shared:
                assert gu[-1]["w"] == E and gu[-1]["n"] == T
                assert gu[-1]["y"][:T].tolist() == list(range(T)) and gu[-1]["out"][:T].tolist() == [T * K + t for t in range(T)]


def test_jobs_decode_skips_missing_picks(orc):
    topi = np.array([[3, -1, 5, -1]], np.int32)
    gu, dn = orc.jobs_decode(topi, 4, E, False)
    assert gu["w"].tolist() == [3, 5] and [j["out"][0] for j in gu] == [0, 2]


def test_jobs_prefill_properties(orc):
    rng = np.random.default_rng(9)
    C = 300
    # skewed routing: some experts take far more than a job's 64 rows
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    topi = np.stack([rng.choice(E, K, replace=False, p=p / p.sum()) for _ in range(C)]).astype(np.int32)
    for shared in (False, True):
        cnt, jbase, gu, dn = orc.jobs_prefill(topi, K, E, shared)
        flat = topi.reshape(-1)
        assert np.array_equal(cnt, np.bincount(flat, minlength=E))
        nj = (cnt + 63) // 64
        assert np.array_equal(jbase, np.concatenate([[0], np.cumsum(nj)[:-1]]))
        assert len(gu) == nj.sum() + (shared * ((C + 63) // 64))
        for e in range(E):
            pairs = []
            for j in range(jbase[e], jbase[e] + nj[e]):
                assert gu[j]["w"] == e and 1 <= gu[j]["n"] <= 64
                pr = gu[j]["out"][: gu[j]["n"]].tolist()
                assert gu[j]["y"][: gu[j]["n"]].tolist() == [q // K for q in pr]
                assert dn[j]["y"][: gu[j]["n"]].tolist() == pr == dn[j]["out"][: gu[j]["n"]].tolist()
                pairs += pr
            assert pairs == np.flatnonzero(flat == e).tolist()   # every pair, in pair-index order
        if shared:
            sh = gu[nj.sum():]
            assert all(j["w"] == E for j in sh)
            assert np.concatenate([j["y"][: j["n"]] for j in sh]).tolist() == list(range(C))


def test_router_logits_prompt_dispatch(orc):
    """sfnx_router_logits' order by chunk size: the VALU order under 512 tokens, the matrix-core order from 512"""
    H, L = 1024, 65
    W = orc.synth(L * H, 25, 0.02).reshape(L, H)
    for T in (orc.ROUTER_MM_MIN_T - 1, orc.ROUTER_MM_MIN_T):
        x = orc.synth(T * H, 26, 1.0).reshape(T, H)
        want = orc.router_logits_mm(W, x) if T >= orc.ROUTER_MM_MIN_T else orc.router_logits(W, x)
        assert np.array_equal(orc.router_logits_prompt(W, x), want)
