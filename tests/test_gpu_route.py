"""GPU parity of activations and routing: q8_1 bytes, router logits, top-k indices and the jobs / permutation are
bit-exact with the oracle; top-k weights (exp) within 1e-6."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sfnx_amd import moe
from sfnx_amd._abi import BIGJOB_INTS, JOB_INTS
from tests.gpu_util import job_array

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows, n", [(1, 2048), (16, 2048), (7, 512), (3, 4096)])
def test_quantize_q8_1_bit_exact(rows, n):
    x = orc.synth(rows * n, 100 + rows, 1.0).reshape(rows, n)
    x[0, :32] = 0.0
    q = torch.empty(rows * n // 32 * 36, dtype=torch.uint8, device="cuda")
    moe.quantize_q8_1(torch.from_numpy(x).cuda(), q)
    assert np.array_equal(q.cpu().numpy(), orc.quantize_q8_1(x))


def route_case(W, x, E, K, shared):
    T, H = x.shape
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    Wd, xd = d(W), d(x)
    logits = torch.empty((T, E + 1), dtype=torch.float32, device="cuda")
    topi = torch.empty((T, K), dtype=torch.int32, device="cuda")
    topw = torch.empty((T, K), dtype=torch.float32, device="cuda")
    nj = T * K + 1
    jg = torch.full((nj * JOB_INTS,), -7, dtype=torch.int32, device="cuda")
    jd = torch.full((nj * JOB_INTS,), -7, dtype=torch.int32, device="cuda")
    njobs = torch.zeros(2, dtype=torch.int32, device="cuda")
    for _ in range(2):   # twice: the block counter must come back to zero
        moe.router_route(Wd, xd, logits, topi, topw, jg, jd, njobs, E, K, shared)
    torch.cuda.synchronize()
    ol = orc.router_logits(W, x)
    assert np.array_equal(logits.cpu().numpy().view(np.uint32), ol.view(np.uint32))
    oi, ow, _ = orc.topk(ol, E, K)
    assert np.array_equal(topi.cpu().numpy(), oi)
    assert np.allclose(topw.cpu().numpy(), ow, rtol=1e-6, atol=1e-7)
    ogu, odn = orc.jobs_decode(oi, K, E, shared)
    n = int(njobs[0])
    assert n == len(ogu) and int(njobs[1]) == 0
    g, dn = job_array(jg)[:n], job_array(jd)[:n]
    for j in range(n):
        c = ogu[j]["n"]
        assert g[j]["w"] == ogu[j]["w"] and g[j]["n"] == c and dn[j]["w"] == odn[j]["w"] and dn[j]["n"] == c
        assert np.array_equal(g[j]["y"][:c], ogu[j]["y"][:c]) and np.array_equal(g[j]["out"][:c], ogu[j]["out"][:c])
        assert np.array_equal(dn[j]["y"][:c], odn[j]["y"][:c]) and np.array_equal(dn[j]["out"][:c], odn[j]["out"][:c])
    return oi


@pytest.mark.parametrize("T", [1, 2, 5, 16])
@pytest.mark.parametrize("shared", [True, False])
def test_router_route_random(T, shared):
    H, E, K = 2048, 512, 10
    W = orc.synth((E + 1) * H, 200, 0.02).reshape(E + 1, H)
    x = orc.synth(T * H, 201 + T, 1.0).reshape(T, H)
    route_case(W, x, E, K, shared)


def test_router_route_exact_ties():
    """duplicated router rows give exactly equal logits: the lower expert wins, as in tools/topk_test.cu"""
    H, E, K = 2048, 512, 10
    W = orc.synth((E + 1) * H, 210, 0.02).reshape(E + 1, H)
    x = orc.synth(4 * H, 211, 1.0).reshape(4, H)
    strong = W[0] * 0 + x[0] * 0.05
    for e in (511, 300, 64, 63, 7, 128, 129):
        W[e] = strong          # seven experts tied for the top
    for e in (200, 201, 450):
        W[e] = strong * 0.5    # three more tied below them
    oi = route_case(W, x, E, K, True)
    assert oi[0].tolist()[:7] == [7, 63, 64, 128, 129, 300, 511]


def test_router_route_all_equal():
    H, E, K = 1024, 256, 8
    W = np.zeros((E + 1, H), np.float32)
    x = orc.synth(3 * H, 212, 1.0).reshape(3, H)
    oi = route_case(W, x, E, K, True)
    assert oi.tolist() == [list(range(K))] * 3


@pytest.mark.parametrize("T, H, L", [(1, 2048, 513), (37, 2048, 513), (300, 2048, 513), (16, 1024, 65),
                                     (40, 2560, 1025), (16, 4096, 129), (300, 4096, 513),
                                     # the matrix-core kernel (512 tokens or more): partial token and row tiles
                                     (512, 2048, 513), (600, 2048, 513), (530, 1024, 65), (777, 2560, 1025),
                                     (520, 4096, 129), (2048, 2048, 513),
                                     # each token tile: 32 (512, 600, 530, 520 tokens), 48 (1000), 64 (1200), 96 (777, 2048)
                                     (1000, 1024, 513), (1200, 1024, 1025)])
def test_router_logits_bit_exact(T, H, L):
    W = orc.synth(L * H, 220, 0.02).reshape(L, H)
    x = orc.synth(T * H, 221, 1.0).reshape(T, H)
    out = torch.empty((T, L), dtype=torch.float32, device="cuda")
    moe.router_logits(torch.from_numpy(W).cuda(), torch.from_numpy(x).cuda(), out)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), orc.router_logits_prompt(W, x).view(np.uint32))


@pytest.mark.parametrize("T, H, L", [(300, 2048, 513), (600, 2048, 513), (777, 2560, 1025), (2048, 4096, 129),
                                     (1000, 1024, 513), (1200, 1024, 1025)])
def test_router_logits_xh(T, H, L):
    """sfnx_router_logits_xh: the same logits as sfnx_router_logits, and xh equal to sfnx_to_f16's, bit for bit"""
    W = torch.from_numpy(orc.synth(L * H, 222, 0.02).reshape(L, H)).cuda()
    x = torch.from_numpy(orc.synth(T * H, 223, 1.0).reshape(T, H)).cuda()
    l0, l1 = (torch.empty((T, L), dtype=torch.float32, device="cuda") for _ in range(2))
    h0, h1 = torch.empty((T, H), dtype=torch.float16, device="cuda"), torch.full((T, H), 7.0, dtype=torch.float16, device="cuda")
    moe.router_logits(W, x, l0)
    moe.to_f16(x, h0)
    moe.router_logits_xh(W, x, l1, h1)
    torch.cuda.synchronize()
    assert torch.equal(l0.view(torch.int32), l1.view(torch.int32))
    assert torch.equal(h0.view(torch.int16), h1.view(torch.int16))


def pf_route_case(logits, E, K, shared):
    C = logits.shape[0]
    cap = C * K // 64 + E + (C + 63) // 64 + 1
    i32 = dict(dtype=torch.int32, device="cuda")
    topi, topw = torch.empty((C, K), **i32), torch.empty((C, K), dtype=torch.float32, device="cuda")
    cnt, jbase = torch.empty(E, **i32), torch.empty(E, **i32)
    jg, jd = torch.zeros(cap * BIGJOB_INTS, **i32), torch.zeros(cap * BIGJOB_INTS, **i32)
    njobs = torch.zeros(2, **i32)
    moe.pf_route(torch.from_numpy(logits).cuda(), topi, topw, cnt, jbase, jg, jd, njobs, E, K, shared)
    torch.cuda.synchronize()
    return topi.cpu().numpy(), topw.cpu().numpy()


def test_topk_near_ties_across_lanes():
    """values a few ulps apart in different lanes (the top-k's fast 32-bit rounds keep only the upper 22 order bits
    beside the index, so these must fall back to the exact rounds), ties, and values straddling zero"""
    E, K = 512, 10
    rng = np.random.default_rng(5)
    rows = []
    for r in range(48):
        row = rng.normal(0, 1, E + 1).astype(np.float32)
        top = np.float32(3.0 + 0.25 * (r % 5))
        idx = rng.choice(E, 14, replace=False)
        if r % 3 == 0:
            idx = np.sort(idx)   # the lower index the smaller value: the truncated key would order these wrongly
        for k, e in enumerate(idx):
            row[e] = np.nextafter(top, np.float32(10.0), dtype=np.float32) if k == 0 else top
            top = np.nextafter(top, np.float32(-10.0), dtype=np.float32) if r % 2 else top
        rows.append(row)
    z = np.full(E + 1, -5.0, np.float32)
    z[[3, 67, 131]] = [np.float32(-0.0), np.float32(0.0), np.float32(1e-45)]
    rows.append(z)
    logits = np.stack(rows)
    topi, topw = pf_route_case(logits, E, K, True)
    oi, ow, _ = orc.topk(logits, E, K)
    assert np.array_equal(topi, oi)
    assert np.allclose(topw, ow, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("C, shared, hot", [(300, True, False), (2048, False, False), (1, True, False),
                                             (4096, True, True), (5000, False, True)])
def test_pf_route_bit_exact(C, shared, hot):
    """hot: every token picks expert 7, so its pairs fill the fill kernel's ranked list exactly (4096) or overflow it
    into the second scan (5000)"""
    E, K = 512, 10
    rng = np.random.default_rng(C)
    logits = rng.normal(0, 1, (C, E + 1)).astype(np.float32)
    logits[:, :E] += (1.1 * -np.log(rng.permutation(E) + 1.0)).astype(np.float32) * 0.8   # skew towards some experts
    if hot:
        logits[:, 7] += 100.0
    if C > 1:
        logits[1, 3:40] = logits[1, 2]   # ties
    cap = C * K // 64 + E + (C + 63) // 64 + 1
    i32 = dict(dtype=torch.int32, device="cuda")
    topi, topw = torch.empty((C, K), **i32), torch.empty((C, K), dtype=torch.float32, device="cuda")
    cnt, jbase = torch.empty(E, **i32), torch.empty(E, **i32)
    jg, jd = torch.zeros(cap * BIGJOB_INTS, **i32), torch.zeros(cap * BIGJOB_INTS, **i32)
    njobs = torch.zeros(2, **i32)
    moe.pf_route(torch.from_numpy(logits).cuda(), topi, topw, cnt, jbase, jg, jd, njobs, E, K, shared)
    torch.cuda.synchronize()
    oi, ow, _ = orc.topk(logits, E, K)
    assert np.array_equal(topi.cpu().numpy(), oi)
    assert np.allclose(topw.cpu().numpy(), ow, rtol=1e-6, atol=1e-7)
    ocnt, ojb, ogu, odn = orc.jobs_prefill(oi, K, E, shared)
    assert np.array_equal(cnt.cpu().numpy(), ocnt) and np.array_equal(jbase.cpu().numpy(), ojb)
    n = int(njobs[0])
    assert n == len(ogu)
    g, d = job_array(jg, True)[:n], job_array(jd, True)[:n]
    for j in range(n):
        c = ogu[j]["n"]
        assert (g[j]["w"], g[j]["n"], d[j]["w"], d[j]["n"]) == (ogu[j]["w"], c, odn[j]["w"], c)
        for f in ("y", "out"):
            assert np.array_equal(g[j][f][:c], ogu[j][f][:c]) and np.array_equal(d[j][f][:c], odn[j][f][:c])
