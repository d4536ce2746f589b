"""The fused decode path (sfnx_moe_decode: three launches a layer) against the unfused entry points (router_route,
moe_gate_up, moe_down, moe_combine), bit for bit, and against the oracle within max relative error 2e-3."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sfnx_amd import moe
from tests.gpu_util import job_array, make_layer, max_rel

pytestmark = pytest.mark.gpu


def bits(t):
    return t.detach().cpu().numpy().view(np.uint32)


def unfused_chain(layers, x, norm, bufs):
    """x += MoE(rmsnorm(x)) per layer with the unfused entry points; returns the last layer's y"""
    xn = torch.empty_like(x)
    y = torch.empty_like(x)
    for L, b in zip(layers, bufs):
        if norm:
            moe.residual_rmsnorm(x, None, xn)
        else:
            xn.copy_(x)
        moe.decode_layer(L, xn, y, b)
        x.add_(y)
    return y


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q5_K, orc.Q4_0, orc.Q5_1, orc.Q8_0])
@pytest.mark.parametrize("T", [1, 3, 16])
def test_fused_layer_equals_unfused(wtype, T):
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=wtype, shared=True)
    L, host = make_layer(shape, 30 + T)
    x0 = torch.from_numpy(orc.synth(T * shape.H, 800 + T, 1.0).reshape(T, shape.H)).cuda()
    b = moe.DecodeBuffers(shape, T)
    xu = x0.clone()
    yu = unfused_chain([L], xu, False, [b])
    f = moe.FusedDecode([L], T)
    xf = x0.clone()
    f(xf, norm=False)
    torch.cuda.synchronize()
    E1, K, P = shape.E + 1, shape.K, T * shape.K
    assert np.array_equal(bits(f.piece("logits", torch.float32, (T, E1))), bits(b.logits))
    assert np.array_equal(f.piece("topi", torch.int32, (T, K)).cpu().numpy(), b.topi.cpu().numpy())
    assert np.array_equal(bits(f.piece("topw", torch.float32, (T, K))), bits(b.topw))
    n = int(f.piece("njobs", torch.int32, (2,))[0])
    assert n == int(b.njobs[0])
    jf = job_array(f.piece("jobs_gu", torch.int32, (P + 1, 34)).reshape(-1))[:n]
    ju = job_array(b.jobs_gu)[:n]
    for a, c in zip(jf, ju):
        assert a["w"] == c["w"] and a["n"] == c["n"]
        assert np.array_equal(a["y"][: a["n"]], c["y"][: c["n"]]) and np.array_equal(a["out"][: a["n"]], c["out"][: c["n"]])
    rows = [p for p in range(P) if b.topi.reshape(-1)[p] >= 0] + list(range(P, P + T))
    gf = f.piece("gu", torch.float32, (P + T, 2 * shape.ff))
    assert np.array_equal(bits(gf[rows]), bits(b.gu[rows]))
    assert np.array_equal(bits(f.piece("y", torch.float32, (T, shape.H))), bits(yu))
    assert np.array_equal(bits(xf), bits(xu))
    # and the oracle
    oy = orc.layer_decode(host, x0.cpu().numpy())[0]
    assert max_rel(yu.cpu().numpy(), oy) < 2e-3


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q5_K, orc.Q4_0, orc.Q5_1, orc.Q8_0])
def test_fused_chain_with_norm_equals_unfused(wtype):
    shape = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=wtype, shared=True)
    layers = [moe.MoeLayer.synthetic(shape, seed=50 + i) for i in range(3)]
    for T in (1, 16):
        x0 = torch.from_numpy(orc.synth(T * shape.H, 900 + T, 1.0).reshape(T, shape.H)).cuda()
        xu = x0.clone()
        yu = unfused_chain(layers, xu, True, [moe.DecodeBuffers(shape, T) for _ in layers])
        f = moe.FusedDecode(layers, T)
        xf = x0.clone()
        f(xf, norm=True)
        torch.cuda.synchronize()
        assert np.array_equal(bits(f.piece("y", torch.float32, (T, shape.H))), bits(yu))
        assert np.array_equal(bits(xf), bits(xu))
        # graph capture and replay give the same result, replay after replay
        xg = x0.clone()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            f(xg, norm=True)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            f(xg, norm=True)
        for _ in range(3):
            xg.copy_(x0)
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(bits(xg), bits(xu))


@pytest.mark.parametrize("wtype, dn_type", [(orc.Q4_K, orc.Q5_K), (orc.Q4_K, orc.Q8_0), (orc.Q5_1, orc.Q4_0)])
def test_mixed_gate_up_and_down_types(wtype, dn_type):
    """gate|up in one type and down in another (the reference's DW per matrix, src/model.cpp:540-606): the fused path
    equals the unfused one bit for bit, and both match the oracle within 2e-3, at the bench shape for 1 and 16 rows"""
    shape = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=wtype, shared=True, dn_wtype=dn_type)
    L, host = make_layer(shape, 61)
    for T in (1, 16):
        x0 = torch.from_numpy(orc.synth(T * shape.H, 810 + T, 1.0).reshape(T, shape.H)).cuda()
        b = moe.DecodeBuffers(shape, T)
        xu = x0.clone()
        yu = unfused_chain([L], xu, False, [b])
        f = moe.FusedDecode([L], T)
        xf = x0.clone()
        f(xf, norm=False)
        torch.cuda.synchronize()
        assert np.array_equal(bits(f.piece("y", torch.float32, (T, shape.H))), bits(yu))
        oy, _, oi, _, ogu, _ = orc.layer_decode(host, x0.cpu().numpy(), nthreads=8)
        assert np.array_equal(b.topi.cpu().numpy(), oi)
        assert max_rel(yu.cpu().numpy(), oy) < 2e-3


@pytest.mark.parametrize("H, E, K, ff, wtype, T", [
    (2560, 1024, 16, 1024, orc.Q4_K, 1), (2560, 1024, 16, 1024, orc.Q4_K, 4), (4096, 128, 4, 512, orc.Q5_K, 1),
    (4096, 128, 4, 512, orc.Q8_0, 16), (1024, 1024, 1, 1024, orc.Q4_0, 2), (2560, 256, 8, 512, orc.Q5_1, 16),
    (2048, 512, 10, 1024, orc.Q4_K, 16)])
def test_fused_decode_edge_shapes(H, E, K, ff, wtype, T):
    """the fused decode's limits: hidden 2560 and 4096, 1024 experts, top-16 and top-1, FF 1024, windows of 1 to 16
    rows: equal to the unfused path bit for bit and to the oracle within 2e-3.  The last case's h (176 pairs of 1024)
    does not fit in the down kernel's LDS, so its down dots read h from memory (the unstaged branch)."""
    shape = moe.LayerShape(H=H, E=E, K=K, ff=ff, wtype=wtype, shared=True)
    L, host = make_layer(shape, 70 + H % 97 + K)
    x0 = torch.from_numpy(orc.synth(T * H, 830 + T + K, 1.0).reshape(T, H)).cuda()
    b = moe.DecodeBuffers(shape, T)
    xu = x0.clone()
    yu = unfused_chain([L], xu, False, [b])
    f = moe.FusedDecode([L], T)
    xf = x0.clone()
    f(xf, norm=False)
    torch.cuda.synchronize()
    assert np.array_equal(bits(f.piece("y", torch.float32, (T, H))), bits(yu))
    assert np.array_equal(bits(xf), bits(xu))
    oy, _, oi, _, _, _ = orc.layer_decode(host, x0.cpu().numpy(), nthreads=8)
    assert np.array_equal(b.topi.cpu().numpy(), oi)
    assert max_rel(yu.cpu().numpy(), oy) < 2e-3


def test_fused_decode_refuses_out_of_range():
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    L, _ = make_layer(shape, 3)
    f = moe.FusedDecode([L], 16)
    with pytest.raises(RuntimeError, match="T out of range"):
        f(torch.zeros((17, 1024), dtype=torch.float32, device="cuda"))


def test_workspace_serves_shorter_windows():
    """one workspace sized for 16 rows, then windows of 4 and 1 rows: each piece's rows hold that window's values
    (the layout does not move with T), equal to the unfused path's"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    L, host = make_layer(shape, 41)
    f = moe.FusedDecode([L], 16)
    for T in (4, 1, 16, 3):
        x0 = torch.from_numpy(orc.synth(T * shape.H, 860 + T, 1.0).reshape(T, shape.H)).cuda()
        b = moe.DecodeBuffers(shape, T)
        xu = x0.clone()
        yu = unfused_chain([L], xu, False, [b])
        xf = x0.clone()
        f(xf, norm=False)
        torch.cuda.synchronize()
        K = shape.K
        assert np.array_equal(f.piece("topi", torch.int32, (T, K)).cpu().numpy(), b.topi.cpu().numpy())
        assert np.array_equal(bits(f.piece("topw", torch.float32, (T, K))), bits(b.topw))
        assert np.array_equal(bits(f.piece("logits", torch.float32, (T, shape.E + 1))), bits(b.logits))
        assert np.array_equal(bits(f.piece("y", torch.float32, (T, shape.H))), bits(yu))
        assert np.array_equal(bits(xf), bits(xu))


def test_fused_chain_drift_against_oracle():
    """config 1's chain, 12 of its stacked layers (x_{l+1} = x_l + MoE_l(rmsnorm(x_l)), each layer's weights seeded
    on their own), through the fused decode against the oracle run layer by layer on the CPU: the last layer's
    router indices equal the oracle's, and its output and the residual stream after 12 layers stay within 2e-3
    (max relative error) of the oracle's chain.  The oracle's rmsnorm is float64 rounded to float32, so the two
    chains' inputs may differ by an ulp from the second layer on: this bounds the drift, it is no bit comparison."""
    shape = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=orc.Q4_K, shared=True)
    NL, eps = 12, 1e-6
    layers, hosts = [], []
    for l in range(NL):
        L, h = make_layer(shape, 500 + l)
        layers.append(L)
        hosts.append(h)
    x0 = orc.synth(shape.H, 4343, 1.0).reshape(1, shape.H)
    f = moe.FusedDecode(layers, 1)
    xf = torch.from_numpy(x0).cuda()
    f(xf, norm=True, eps=eps)
    torch.cuda.synchronize()
    x = x0.astype(np.float32)
    for h in hosts:
        ss = np.sum(x.astype(np.float64) ** 2, axis=1)
        r = (1.0 / np.sqrt(ss / shape.H + eps)).astype(np.float32)
        xn = (x * r[:, None]).astype(np.float32)
        oy, ol, oi, ow, ogu, opart = orc.layer_decode(h, xn, nthreads=8)
        x = (x + oy).astype(np.float32)
    assert np.array_equal(f.piece("topi", torch.int32, (1, shape.K)).cpu().numpy(), oi)
    assert max_rel(f.piece("y", torch.float32, (1, shape.H)).cpu().numpy(), oy) < 2e-3
    assert max_rel(xf.cpu().numpy(), x) < 2e-3


@pytest.mark.parametrize("T", [1, 4])
def test_fused_window_with_no_picks(T):
    """rows whose logits are all NaN pick nothing: with no shared expert the window has no job at all, and the fused
    decode's kernels (whose gate|up blocks map to jobs modulo the job count) still finish, and agree with the unfused
    path: every pick -1, a zero job count, y = 0"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=False)
    L, _ = make_layer(shape, 71)
    x0 = torch.full((T, shape.H), float("nan"), dtype=torch.float32, device="cuda")
    b = moe.DecodeBuffers(shape, T)
    y = torch.empty_like(x0)
    moe.decode_layer(L, x0, y, b)
    f = moe.FusedDecode([L], T)
    xf = x0.clone()
    f(xf, norm=False)
    torch.cuda.synchronize()
    assert (b.topi == -1).all() and int(b.njobs[0]) == 0
    assert (f.piece("topi", torch.int32, (T, shape.K)) == -1).all()
    assert int(f.piece("njobs", torch.int32, (2,))[0]) == 0
    assert (y == 0).all() and (f.piece("y", torch.float32, (T, shape.H)) == 0).all()
