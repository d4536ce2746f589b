"""GPU parity of the expert kernels and the whole layer against the oracle, through the C ABI.

Bit-exact: gate|up outputs (integer dots and the fp32 combine in the oracle's order), top-k indices, jobs.
Within tolerance: down outputs and the layer output, because silu / sigmoid / softmax use the device's expf where the
oracle uses libm's (the reference itself uses fast-math __expf); the bar is a max relative error of 2e-3 (fp32 accumulation),
measured as max |err| / max |ref| over each output.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sfnx_amd import moe
from tests.gpu_util import make_layer, max_rel

pytestmark = pytest.mark.gpu
TOL = 2e-3


def routed_rows(topi, T, K, shared):
    rows = [p for p in range(T * K) if topi.reshape(-1)[p] >= 0]
    return rows + ([T * K + t for t in range(T)] if shared else [])


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q5_K, orc.Q4_0, orc.Q5_1, orc.Q8_0])
@pytest.mark.parametrize("T", [1, 3, 16])
def test_decode_layer_small(wtype, T):
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=wtype, shared=True)
    L, host = make_layer(shape, 3 + T + wtype)
    x = orc.synth(T * shape.H, 500 + T, 1.0).reshape(T, shape.H)
    y = torch.empty((T, shape.H), dtype=torch.float32, device="cuda")
    b = moe.DecodeBuffers(shape, T)
    moe.decode_layer(L, torch.from_numpy(x).cuda(), y, b)
    torch.cuda.synchronize()
    oy, ol, oi, ow, ogu, opart = orc.layer_decode(host, x)
    assert np.array_equal(b.topi.cpu().numpy(), oi)
    rows = routed_rows(oi, T, shape.K, True)
    gu = b.gu.cpu().numpy()[rows]
    assert np.array_equal(gu.view(np.uint32), ogu[rows].view(np.uint32)), "gate|up not bit-exact"
    part = b.part.cpu().numpy()[rows]
    assert max_rel(part, opart[rows]) < TOL
    exact = np.mean(part == opart[rows])
    assert exact > 0.5, exact
    assert max_rel(y.cpu().numpy(), oy) < TOL


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q5_K, orc.Q4_0, orc.Q5_1, orc.Q8_0])
def test_prefill_q8_layer(wtype):
    """the BigJob kernels (prompt path, q8_1 arithmetic) on a skewed chunk: same per-pair arithmetic as decode"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=wtype, shared=True)
    L, host = make_layer(shape, 60 + wtype)
    C = 200
    x = orc.synth(C * shape.H, 600, 1.0).reshape(C, shape.H)
    # one token repeated: a job fills all its 64 rows and runs several passes through the row
    x[100:180] = x[99]
    y = torch.empty((C, shape.H), dtype=torch.float32, device="cuda")
    b = moe.PrefillBuffers(shape, C)
    moe.prefill_layer_q8(L, torch.from_numpy(x).cuda(), y, b)
    torch.cuda.synchronize()
    oy, ol, oi, ow, ogu, opart = orc.layer_decode(host, x, nthreads=8, prompt=True)
    assert np.array_equal(b.topi.cpu().numpy(), oi)
    assert int(b.cnt.max()) > 64
    rows = routed_rows(oi, C, shape.K, True)
    assert np.array_equal(b.gu.cpu().numpy()[rows].view(np.uint32), ogu[rows].view(np.uint32))
    assert max_rel(b.part.cpu().numpy()[rows], opart[rows]) < TOL
    assert max_rel(y.cpu().numpy(), oy) < TOL


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q5_K, orc.Q4_0, orc.Q5_1, orc.Q8_0])
def test_decode_layer_baseline_shapes(wtype):
    """The benchmark layer shape (configs 0/1/4): hidden 2048, 512 experts x FF 512, top-10 + shared, one token and a 16-row window"""
    shape = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=wtype, shared=True)
    L, host = make_layer(shape, 1)
    for T in (1, 16):
        x = orc.synth(T * shape.H, 700 + T, 1.0).reshape(T, shape.H)
        y = torch.empty((T, shape.H), dtype=torch.float32, device="cuda")
        b = moe.DecodeBuffers(shape, T)
        moe.decode_layer(L, torch.from_numpy(x).cuda(), y, b)
        torch.cuda.synchronize()
        oy, ol, oi, ow, ogu, opart = orc.layer_decode(host, x, nthreads=8)
        assert np.array_equal(b.logits.cpu().numpy().view(np.uint32), ol.view(np.uint32))
        assert np.array_equal(b.topi.cpu().numpy(), oi)
        rows = routed_rows(oi, T, shape.K, True)
        assert np.array_equal(b.gu.cpu().numpy()[rows].view(np.uint32), ogu[rows].view(np.uint32))
        assert max_rel(y.cpu().numpy(), oy) < TOL


def test_combine_matches_oracle_weighted_sum():
    T, H, E, K = 4, 2048, 512, 10
    rng = np.random.default_rng(3)
    part = rng.normal(0, 1, (T * K + T, H)).astype(np.float32)
    topw = rng.random((T, K)).astype(np.float32)
    topi = rng.integers(0, E, (T, K)).astype(np.int32)
    topi[2, 4] = -1
    logits = rng.normal(0, 2, (T, E + 1)).astype(np.float32)
    d = lambda a: torch.from_numpy(a).cuda()
    y = torch.empty((T, H), dtype=torch.float32, device="cuda")
    moe.moe_combine(d(part), d(topw), d(topi), d(logits), y, E, K, True)
    sig = 1 / (1 + np.exp(-logits[:, E].astype(np.float64)))
    w = np.where(topi >= 0, topw, 0).astype(np.float64)
    want = np.einsum("tk,tkh->th", w, part[: T * K].reshape(T, K, H)) + sig[:, None] * part[T * K:]
    assert max_rel(y.cpu().numpy(), want) < 1e-6
