"""The matrix-core prompt path (moe_gate_up_mma, swiglu_h16, moe_down_mma) against float64 products of the f16
weights and f16 activations, sampled as tools/moe_mma_bench.cu:197-220 samples them (max error over the sample's largest
value), and the whole f16 layer against a float64 restatement of it.  Tolerance: 2e-3 max relative error, the stated bound for fp32 accumulation (fp32 accumulation
measures ~1e-6 here)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sfnx_amd import moe
from tests.gpu_util import job_array, make_layer, max_rel

pytestmark = pytest.mark.gpu


def f16_of(a):
    return np.asarray(a, np.float32).astype(np.float16)


def expert_rows(host, e, down):
    rb = orc.row_bytes(host.dn_type if down else host.type, host.ff if down else host.H)
    if down:
        return host.dn_w[e * host.dn_stride:(e + 1) * host.dn_stride], rb
    return host.gu_w[e * host.gu_stride:(e + 1) * host.gu_stride], rb


class F16Experts:
    """an expert's matrices dequantized to f16 (the oracle's f16 dequantization, src/moe_mma.cuh:56-62 and 121-216),
    held as float64 for the float64 products; the last expert's only (callers visit each expert's work together)"""

    def __init__(self, host):
        self.host, self.cache = host, {}

    def __call__(self, e, down):
        k = (e, down)
        if k not in self.cache:
            self.cache = {c: v for c, v in self.cache.items() if c[0] == e}
            h = self.host
            w, _ = expert_rows(h, e, down)
            t, rows, cols = (h.dn_type, h.H, h.ff) if down else (h.type, 2 * h.ff, h.H)
            self.cache[k] = orc.dequant_f16(t, w, rows, cols).view(np.float16).astype(np.float64).reshape(rows, cols)
        return self.cache[k]


def run_prefill(shape, seed, C, dup=False, bias=None):
    L, host = make_layer(shape, seed)
    x = orc.synth(C * shape.H, seed + 7, 1.0).reshape(C, shape.H)
    if dup:
        x[40:140] = x[39]   # one token 100 times: its experts' jobs fill all 64 rows
    xd = torch.from_numpy(x).cuda()
    y = torch.empty_like(xd)
    b = moe.PrefillBuffers(shape, C)
    moe.prefill_route(L, xd, b, None if bias is None else torch.from_numpy(bias).cuda())
    moe.prefill_experts_mma(L, xd, y, b)
    torch.cuda.synchronize()
    return L, host, x, y.cpu().numpy(), b


def check_sampled(host, x, b, nsample, rng):
    s = host
    topi = b.topi.cpu().numpy()
    C, K = topi.shape
    P = C * K
    gu = b.gu.cpu().numpy()
    h16 = b.h16.cpu().numpy()
    part = b.part.cpu().numpy()
    x16 = f16_of(x)
    eg, mg, ed, md = 0.0, 0.0, 0.0, 0.0
    f16w = F16Experts(host)
    ps = [int(p) for p in rng.integers(0, P + C, nsample)]
    for p in sorted(ps, key=lambda p: int(topi.reshape(-1)[p]) if p < P else s.E):   # each expert's samples together
        if p < P:
            e, t = int(topi.reshape(-1)[p]), p // K
        else:
            e, t = s.E, p - P
        ref = f16w(e, False) @ x16[t].astype(np.float64)
        mg = max(mg, np.abs(ref).max())
        eg = max(eg, np.abs(ref - gu[p]).max())
        refd = f16w(e, True) @ h16[p].astype(np.float64)
        md = max(md, np.abs(refd).max())
        ed = max(ed, np.abs(refd - part[p]).max())
        # h16 is f16(silu(g) u) of the kernel's own gate|up row
        hh = orc.swiglu_h16(gu[p], s.ff).view(np.float16).astype(np.float32)
        assert np.max(np.abs(hh - h16[p].astype(np.float32))) <= 2 ** -10 * np.max(np.abs(hh)) + 1e-7
    return eg / mg, ed / md


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q5_K, orc.Q4_0, orc.Q5_1, orc.Q8_0])
def test_mma_small_layer_with_full_jobs(wtype):
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=wtype, shared=True)
    L, host, x, y, b = run_prefill(shape, 70 + wtype, 200, dup=True)
    assert int(b.cnt.max()) > 64          # some experts split over several 64-row jobs
    jobs = job_array(b.jobs_gu, True)[: int(b.njobs[0])]
    assert (jobs["n"] == 64).any() and (jobs["n"] < 33).any()
    eg, ed = check_sampled(host, x, b, 40, np.random.default_rng(1))
    assert eg < 2e-3 and ed < 2e-3, (eg, ed)
    # the layer: the combine of the kernel's own rows
    topi, topw = b.topi.cpu().numpy(), b.topw.cpu().numpy().astype(np.float64)
    part = b.part.cpu().numpy().astype(np.float64)
    C, K = topi.shape
    lg = b.logits.cpu().numpy()
    sig = 1 / (1 + np.exp(-lg[:, shape.E].astype(np.float64)))
    want = np.einsum("tk,tkh->th", topw, part[: C * K].reshape(C, K, -1)) + sig[:, None] * part[C * K:]
    assert max_rel(y, want) < 1e-5


def layer_rows_f64(host, shape, x16, lg, oi, ow, rows):
    """float64 restatement of the f16 layer for the given tokens: per pick (and the shared expert), the f16 weights
    times the f16 activations (float64 sums), f16(silu(g) u), the f16 down weights times that, weighted by the routing"""
    out = np.zeros((len(rows), shape.H))
    f16w = F16Experts(host)
    work = []
    for i, t in enumerate(rows):
        picks = [(int(e), float(w)) for e, w in zip(oi[t], ow[t]) if e >= 0]
        picks.append((shape.E, 1 / (1 + np.exp(-float(lg[t, shape.E])))))
        work += [(e, w, i, t) for e, w in picks]
    for e, w, i, t in sorted(work):   # each expert dequantized once
        gu = f16w(e, False) @ x16[t].astype(np.float64)
        hh = orc.swiglu_h16(gu.astype(np.float32), shape.ff).view(np.float16).astype(np.float64)
        out[i] += w * (f16w(e, True) @ hh)
    return out


def check_prompt_routing(b, logits, shape):
    """the prompt path's top-k and BigJobs against the oracle's on the same logits, exactly"""
    E, K = shape.E, shape.K
    oi, ow, _ = orc.topk(logits, E, K)
    assert np.array_equal(b.topi.cpu().numpy(), oi)
    assert np.allclose(b.topw.cpu().numpy(), ow, rtol=1e-6, atol=1e-7)
    ocnt, ojb, ogu, odn = orc.jobs_prefill(oi, K, E, shape.shared)
    assert np.array_equal(b.cnt.cpu().numpy(), ocnt) and np.array_equal(b.jbase.cpu().numpy(), ojb)
    n = int(b.njobs[0])
    assert n == len(ogu)
    g, d = job_array(b.jobs_gu, True)[:n], job_array(b.jobs_dn, True)[:n]
    for j in range(n):
        c = ogu[j]["n"]
        assert (g[j]["w"], g[j]["n"], d[j]["w"], d[j]["n"]) == (ogu[j]["w"], c, odn[j]["w"], c)
        for f in ("y", "out"):
            assert np.array_equal(g[j][f][:c], ogu[j][f][:c]) and np.array_equal(d[j][f][:c], odn[j][f][:c])
    return oi, ow


def test_mma_baseline_prefill_shape():
    """The benchmark prefill shape (config 3): 2048 tokens, hidden 2048, 512 experts x FF 512, top-10 + shared,
    Zipf-skewed routing.  The router logits bit for bit and the top-k and BigJobs exactly against the oracle on the
    biased logits; 400 sampled (pair, gate|up row set) and (pair, down row set) products within 2e-3 of float64 (the
    sample size of tools/moe_mma_bench.cu:197-220); the whole layer (fused gate|up + SwiGLU, down, combine) for 64
    tokens within 2e-3 of its float64 restatement"""
    shape = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=orc.Q4_K, shared=True)
    rank = np.random.default_rng(7).permutation(512) + 1
    bias = (0.125 * -1.1 * np.log(rank)).astype(np.float32)
    L, host, x, y, b = run_prefill(shape, 3, 2048, bias=bias)
    assert 150 < int(b.cnt.max()) < 260
    lg = orc.router_logits_prompt(host.W, x)
    got_lg = b.logits.cpu().numpy()
    lg_biased = lg.copy()
    lg_biased[:, : shape.E] += bias
    assert np.array_equal(got_lg.view(np.uint32), lg_biased.view(np.uint32))
    oi, ow = check_prompt_routing(b, lg_biased, shape)
    eg, ed = check_sampled(host, x, b, 400, np.random.default_rng(2))
    assert eg < 2e-3 and ed < 2e-3, (eg, ed)
    # the whole layer as the prompt path runs it
    xd = torch.from_numpy(x).cuda()
    yl = torch.empty_like(xd)
    b2 = moe.PrefillBuffers(shape, 2048)
    moe.prefill_layer_mma(L, xd, yl, b2, torch.from_numpy(bias).cuda())
    torch.cuda.synchronize()
    rows = list(np.random.default_rng(5).choice(2048, 64, replace=False))
    want = layer_rows_f64(host, shape, f16_of(x), lg_biased, oi, ow, rows)
    assert max_rel(yl.cpu().numpy()[rows], want) < 2e-3


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q5_K, orc.Q4_0, orc.Q5_1, orc.Q8_0])
def test_gate_up_swiglu_fused_equals_two_calls(wtype):
    """sfnx_moe_gate_up_swiglu_mma against moe_gate_up_mma + swiglu_h16 on the same jobs: bit for bit"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=wtype, shared=True)
    L, host, x, y, b = run_prefill(shape, 90 + wtype, 200, dup=True)
    s = shape
    fused = torch.full_like(b.h16, 7.0)
    moe.moe_gate_up_swiglu_mma(L.gu_w, L.gu_stride, s.wtype, s.H, s.ff, b.jobs_gu, b.njobs, b.cap, b.xh, fused)
    torch.cuda.synchronize()
    P = int(b.topi.numel()) + 200
    assert torch.equal(fused[:P].view(torch.int16), b.h16[:P].view(torch.int16))


def test_verify_window_whole_layer():
    """config 2's shape: 96 rows through the whole layer on the prompt path (fused gate|up + SwiGLU): routing and
    BigJobs against the oracle exactly, and every one of the 96 rows against the float64 restatement of the f16 layer"""
    shape = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=orc.Q4_K, shared=True)
    L, host = make_layer(shape, 11)
    C = 96
    x = orc.synth(C * shape.H, 18, 1.0).reshape(C, shape.H)
    xd = torch.from_numpy(x).cuda()
    y = torch.empty_like(xd)
    b = moe.PrefillBuffers(shape, C)
    moe.prefill_layer_mma(L, xd, y, b)
    torch.cuda.synchronize()
    lg = orc.router_logits_prompt(host.W, x)
    assert np.array_equal(b.logits.cpu().numpy().view(np.uint32), lg.view(np.uint32))
    oi, ow = check_prompt_routing(b, lg, shape)
    yo = y.cpu().numpy()
    want = layer_rows_f64(host, shape, f16_of(x), lg, oi, ow, range(C))
    for t in range(C):
        assert np.abs(yo[t] - want[t]).max() <= 2e-3 * np.abs(want[t]).max(), t


def test_q8_0_prefill_4096():
    """config 4's prompt chunk as the bench runs it: 4096 tokens through Q8_0 experts on the matrix cores with the
    bench's Zipf-skewed routing.  The router logits bit for bit and the top-k and BigJobs exactly against the oracle on
    the biased logits; 400 sampled (pair, gate|up row set) and (pair, down row set) products within 2e-3 of float64;
    the whole layer (fused gate|up + SwiGLU, down, combine) for 64 tokens within 2e-3 of its float64 restatement"""
    shape = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=orc.Q8_0, shared=True)
    rank = np.random.default_rng(7).permutation(512) + 1
    bias = (0.125 * -1.1 * np.log(rank)).astype(np.float32)
    C = 4096
    L, host, x, y, b = run_prefill(shape, 23, C, bias=bias)
    assert int(b.cnt.max()) > 300   # the skew's hottest experts take several 64-row jobs
    lg = orc.router_logits_prompt(host.W, x)
    lg[:, : shape.E] += bias
    assert np.array_equal(b.logits.cpu().numpy().view(np.uint32), lg.view(np.uint32))
    oi, ow = check_prompt_routing(b, lg, shape)
    eg, ed = check_sampled(host, x, b, 400, np.random.default_rng(3))
    assert eg < 2e-3 and ed < 2e-3, (eg, ed)
    xd = torch.from_numpy(x).cuda()
    yl = torch.empty_like(xd)
    b2 = moe.PrefillBuffers(shape, C)
    moe.prefill_layer_mma(L, xd, yl, b2, torch.from_numpy(bias).cuda())
    torch.cuda.synchronize()
    rows = list(np.random.default_rng(6).choice(C, 64, replace=False))
    want = layer_rows_f64(host, shape, f16_of(x), lg, oi, ow, rows)
    assert max_rel(yl.cpu().numpy()[rows], want) < 2e-3


@pytest.mark.parametrize("wtype, dn_type", [(orc.Q4_K, orc.Q5_K), (orc.Q4_0, orc.Q8_0)])
def test_mma_mixed_gate_up_and_down_types(wtype, dn_type):
    """gate|up of one type, down of another, on the matrix cores: sampled rows within 2e-3 of float64 products"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=wtype, shared=True, dn_wtype=dn_type)
    L, host, x, y, b = run_prefill(shape, 77, 200, dup=True)
    eg, ed = check_sampled(host, x, b, 30, np.random.default_rng(4))
    assert eg < 2e-3 and ed < 2e-3, (eg, ed)


@pytest.mark.parametrize("C", [1, 17, 1000])
def test_mma_extreme_skew_and_tiny_chunks(C):
    """every token routed to the same 6 experts (a bias of +100 on their logits): each takes C rows, up to 16 BigJobs
    of one expert in a row; and chunks of 1 and 17 tokens.  Routing against the oracle's on the biased logits, sampled
    pairs within 2e-3 of float64, the combine of the kernel's own rows"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    L, host = make_layer(shape, 123)
    x = orc.synth(C * shape.H, 124 + C, 1.0).reshape(C, shape.H)
    xd = torch.from_numpy(x).cuda()
    bias = np.zeros(shape.E, np.float32)
    bias[[3, 9, 17, 33, 40, 63]] = 100.0
    y = torch.empty_like(xd)
    b = moe.PrefillBuffers(shape, C)
    moe.prefill_route(L, xd, b, torch.from_numpy(bias).cuda())
    moe.prefill_experts_mma(L, xd, y, b)
    torch.cuda.synchronize()
    lg = orc.router_logits_prompt(host.W, x)
    lg[:, : shape.E] += bias
    oi, ow, _ = orc.topk(lg, shape.E, shape.K)
    assert np.array_equal(b.topi.cpu().numpy(), oi)
    assert sorted(set(oi.reshape(-1).tolist())) == [3, 9, 17, 33, 40, 63]
    cnt = b.cnt.cpu().numpy()
    assert cnt[[3, 9, 17, 33, 40, 63]].tolist() == [C] * 6 and cnt.sum() == 6 * C
    jobs = job_array(b.jobs_gu, True)[: int(b.njobs[0])]
    assert len(jobs) == 6 * ((C + 63) // 64) + (C + 63) // 64
    eg, ed = check_sampled(host, x, b, min(40, 7 * C), np.random.default_rng(C))
    assert eg < 2e-3 and ed < 2e-3, (eg, ed)
    topw = b.topw.cpu().numpy().astype(np.float64)
    part = b.part.cpu().numpy().astype(np.float64)
    sig = 1 / (1 + np.exp(-b.logits.cpu().numpy()[:, shape.E].astype(np.float64)))
    want = np.einsum("tk,tkh->th", topw, part[: C * shape.K].reshape(C, shape.K, -1)) + sig[:, None] * part[C * shape.K:]
    assert max_rel(y.cpu().numpy(), want) < 1e-5


@pytest.mark.parametrize("H, ff, wtype", [(4096, 512, orc.Q4_K), (2560, 1024, orc.Q8_0), (4096, 1024, orc.Q5_1)])
def test_mma_wide_hidden(H, ff, wtype):
    """the prompt path at hidden 2560 and 4096 and FF 1024 (the router's widest LDS form, the MMA's 5 and 8 runs a
    row): routing against the oracle, sampled pairs within 2e-3 of float64"""
    shape = moe.LayerShape(H=H, E=64, K=6, ff=ff, wtype=wtype, shared=True)
    L, host, x, y, b = run_prefill(shape, 200 + H % 97, 150)
    lg = orc.router_logits_prompt(host.W, x)
    oi, _, _ = orc.topk(lg, shape.E, shape.K)
    assert np.array_equal(b.topi.cpu().numpy(), oi)
    eg, ed = check_sampled(host, x, b, 24, np.random.default_rng(H))
    assert eg < 2e-3 and ed < 2e-3, (eg, ed)
