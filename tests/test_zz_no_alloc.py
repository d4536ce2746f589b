"""sfnx_moe_decode_noalloc (the decode with the library's own device scratch, for callers that cannot allocate)
through the C ABI, against sfnx_moe_decode2 with a caller's workspace: bit for bit, on two calls in a row, the second
with a smaller input (fewer rows and a smaller layer), so that the scratch's previous contents cannot leak in."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sfnx_amd import _abi, moe
from sfnx_amd._abi import check, lib

pytestmark = pytest.mark.gpu


def noalloc(layers, x, norm=True, eps=1e-6):
    s = layers[0].s
    table = (_abi.LayerW * len(layers))(*[
        _abi.LayerW(L.W.data_ptr(), L.gu_w.data_ptr(), L.gu_stride, L.dn_w.data_ptr(), L.dn_stride) for L in layers])
    check(lib().sfnx_moe_decode_noalloc(C.cast(table, C.c_void_p), len(layers), s.wtype, s.dn_type, s.H, s.E, s.K, s.ff,
                                        int(s.shared), x.data_ptr(), x.shape[0], int(norm), eps,
                                        torch.cuda.current_stream().cuda_stream))


def with_workspace(layers, x, norm=True):
    f = moe.FusedDecode(layers, x.shape[0])
    f(x, norm=norm)


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q8_0])
def test_noalloc_equals_workspace_decode(wtype):
    big = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=wtype, shared=True)
    small = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=wtype, shared=True)
    for shape, T, nl, seed in ((big, 16, 2, 500), (small, 4, 3, 600), (big, 1, 2, 700)):
        layers = [moe.MoeLayer.synthetic(shape, seed=seed + i) for i in range(nl)]
        x0 = torch.from_numpy(orc.synth(T * shape.H, seed, 1.0).reshape(T, shape.H)).cuda()
        xa, xb = x0.clone(), x0.clone()
        with_workspace(layers, xa)
        noalloc(layers, xb)
        torch.cuda.synchronize()
        assert torch.isfinite(xa).all()
        assert np.array_equal(xa.cpu().numpy().view(np.uint32), xb.cpu().numpy().view(np.uint32)), (shape, T)


def test_noalloc_refuses_bad_arguments():
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    layers = [moe.MoeLayer.synthetic(shape, seed=800)]
    with pytest.raises(RuntimeError, match="T out of range"):
        noalloc(layers, torch.zeros((17, 1024), dtype=torch.float32, device="cuda"))


def test_noalloc_refuses_a_call_that_overlaps_another_streams():
    """two streams on one GPU share the scratch array: a call on stream B while stream A's call is still queued behind
    long work is refused with a clear error (instead of racing on the array); once A's call has finished, B's runs and
    equals the workspace path"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    layers = [moe.MoeLayer.synthetic(shape, seed=900)]
    x0 = torch.from_numpy(orc.synth(2 * shape.H, 901, 1.0).reshape(2, shape.H)).cuda()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    m = torch.randn(4096, 4096, device="cuda")
    torch.cuda.synchronize()
    xa, xb = x0.clone(), x0.clone()
    with torch.cuda.stream(sa):
        for _ in range(40):   # ~tens of ms of work ahead of A's call
            m = m @ m * 1e-3
        noalloc(layers, xa)
    with torch.cuda.stream(sb):
        with pytest.raises(RuntimeError, match="another stream still runs"):
            noalloc(layers, xb)
    torch.cuda.synchronize()
    with torch.cuda.stream(sb):
        noalloc(layers, xb)
    xw = x0.clone()
    with_workspace(layers, xw)
    torch.cuda.synchronize()
    assert np.array_equal(xa.cpu().numpy().view(np.uint32), xw.cpu().numpy().view(np.uint32))
    assert np.array_equal(xb.cpu().numpy().view(np.uint32), xw.cpu().numpy().view(np.uint32))
