"""The hyper-connection read (sfnx_hc_read; src/hc.cuh k_hc) against the oracle (orc_hc_read) on the same inputs:
the slices' square sums and partial down / inject dots bit-exact; lo (int8 after silu) and mixed within the bar of
every output after silu / sigmoid (2e-3 max relative error; the device's expf and libm's may differ in the last bit);
xq bit-exact as the q8_1 of the kernel's own mixed; R' written back.  And the read feeding the fused decode: K1's q8_1
of mixed (no norm) equals the read's xq."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sfnx_amd import moe
from tests.gpu_util import make_layer, max_rel
from tests.hc_util import hc_inputs

pytestmark = pytest.mark.gpu


def run(N, HC, LR, T, seed, fold, inject=True):
    w, R, bo, inj = hc_inputs(N, HC, LR, T, seed, inject)
    h = moe.HcRead(N, HC, LR, w["w_norm"], w["dq"], w["dd"], w["uq"], w["ud"], w["w_inj"])
    Rd = torch.from_numpy(R).cuda()
    mixed = torch.empty((T, N), dtype=torch.float32, device="cuda")
    xq = torch.empty(T * (N // 32) * 36, dtype=torch.uint8, device="cuda")
    injo = torch.zeros((T, HC), dtype=torch.float32, device="cuda")
    h(Rd, mixed, xq, torch.from_numpy(bo).cuda() if fold else None, torch.from_numpy(inj).cuda() if fold else None,
      injo if inject else None)
    torch.cuda.synchronize()
    ow = orc.HcWeights(N, HC, LR, w["w_norm"], w["dq"], w["dd"], w["uq"], w["ud"], w["w_inj"])
    ref = orc.hc_read(ow, R, bo if fold else None, inj if fold else None)
    return h, Rd, mixed, xq, injo, ref


@pytest.mark.parametrize("N,HC,LR", [(2560, 4, 320), (512, 2, 96), (1024, 8, 256), (512, 1, 512)])
@pytest.mark.parametrize("T", [1, 3, 5, 16])
def test_hc_read_against_oracle_no_fold(N, HC, LR, T):
    h, Rd, mixed, xq, injo, (om, oi, oxq, oR, opart, ossp) = run(N, HC, LR, T, 100 + T + N, fold=False)
    NS = HC * N // 512
    part = h.piece("part", torch.float32, (T, NS, LR + HC)).cpu().numpy()
    ssp = h.piece("ssp", torch.float32, (T, NS)).cpu().numpy()
    assert np.array_equal(ssp.view(np.uint32), ossp.view(np.uint32)), "square sums not bit-exact"
    assert np.array_equal(part.view(np.uint32), opart.view(np.uint32)), "partial dots not bit-exact"
    assert np.array_equal(Rd.cpu().numpy(), oR)   # no fold: R untouched
    assert max_rel(injo.cpu().numpy(), oi) < 1e-6
    m = mixed.cpu().numpy()
    assert max_rel(m, om) < 2e-3
    assert np.mean(m == om) > 0.9
    ref_xq = torch.empty_like(xq)
    moe.quantize_q8_1(mixed, ref_xq)
    torch.cuda.synchronize()
    assert torch.equal(xq, ref_xq)


@pytest.mark.parametrize("T", [1, 4])
def test_hc_read_with_fold(T):
    h, Rd, mixed, xq, injo, (om, oi, oxq, oR, opart, ossp) = run(2560, 4, 320, T, 300 + T, fold=True)
    assert max_rel(Rd.cpu().numpy(), oR) < 1e-6            # R' written back (its sigmoid through expf)
    assert max_rel(mixed.cpu().numpy(), om) < 2e-3
    assert max_rel(injo.cpu().numpy(), oi) < 1e-4


def test_hc_read_without_inject_rows():
    h, Rd, mixed, xq, injo, (om, oi, *_rest) = run(512, 4, 64, 3, 7, fold=True, inject=False)
    assert (injo.cpu().numpy() == 0).all()
    assert max_rel(mixed.cpu().numpy(), om) < 2e-3


def test_hc_read_feeds_the_decode():
    """mixed through a MoE layer: the fused decode's own q8_1 of its input (norm off) is the read's xq, bit for bit"""
    N, HC, LR, T = 1024, 4, 320, 3
    h, Rd, mixed, xq, injo, ref = run(N, HC, LR, T, 41, fold=True)
    shape = moe.LayerShape(H=N, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    L, host = make_layer(shape, 42)
    f = moe.FusedDecode([L], T)
    x = mixed.clone()
    f(x, norm=False)
    torch.cuda.synchronize()
    assert torch.equal(f.piece("xq", torch.uint8, (T * (N // 32) * 36,)), xq)
    oy = orc.layer_decode(host, mixed.cpu().numpy())[0]
    assert max_rel(f.piece("y", torch.float32, (T, N)).cpu().numpy(), oy) < 2e-3


def test_hc_read_refusals():
    w, R, bo, inj = hc_inputs(512, 4, 64, 1, 1)
    h = moe.HcRead(512, 4, 64, w["w_norm"], w["dq"], w["dd"], w["uq"], w["ud"], w["w_inj"])
    Rd = torch.from_numpy(R).cuda()
    mixed = torch.empty((1, 512), dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="inj_prev"):
        h(Rd, mixed, bo=torch.from_numpy(bo).cuda())
    Rd2 = torch.zeros((17, 2048), dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="T out of range"):
        h(Rd2, torch.empty((17, 512), dtype=torch.float32, device="cuda"))


@pytest.mark.parametrize("T", [1, 5])
def test_hc_read_graph_replays(T):
    """the read captured in a HIP graph (as the bench times it): every replay, with eager work between them, gives the
    eager mixed, xq and inject bit for bit (no fold, so R stays as it is)"""
    N, HC, LR = 2560, 4, 320
    w, R, bo, inj = hc_inputs(N, HC, LR, T, 500 + T)
    h = moe.HcRead(N, HC, LR, w["w_norm"], w["dq"], w["dd"], w["uq"], w["ud"], w["w_inj"])
    Rd = torch.from_numpy(R).cuda()
    mixed = torch.empty((T, N), dtype=torch.float32, device="cuda")
    xq = torch.empty(T * (N // 32) * 36, dtype=torch.uint8, device="cuda")
    injo = torch.zeros((T, HC), dtype=torch.float32, device="cuda")
    h(Rd, mixed, xq, inject=injo)
    torch.cuda.synchronize()
    want = (mixed.clone(), xq.clone(), injo.clone())
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        h(Rd, mixed, xq, inject=injo)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        h(Rd, mixed, xq, inject=injo)
    for i in range(3):
        mixed.fill_(float(i))
        xq.zero_()
        injo.fill_(-1.0)
        h.ws.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(mixed, want[0]) and torch.equal(xq, want[1]) and torch.equal(injo, want[2]), i
