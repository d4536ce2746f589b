"""Experts reached through per-expert pointer tables (the reference's DW::ep / moe_expert, src/moe_w.cuh:2-9,
src/model.hpp:85-86): a store with stride 0 is a device table of each expert's matrix.  Every path that reads experts
(the fused decode, the unfused decode calls, the prompt path's matrix-core and q8 calls) gives the same bits through a
table over moved, shuffled copies of the matrices as through the strided store."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sfnx_amd import moe
from tests.gpu_util import make_layer, tabled

pytestmark = pytest.mark.gpu


def bits(t):
    return t.detach().cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("wtype, dn_type", [(orc.Q4_K, orc.Q4_K), (orc.Q8_0, orc.Q8_0), (orc.Q4_K, orc.Q5_1)])
@pytest.mark.parametrize("T", [1, 16])
def test_decode_through_tables(wtype, dn_type, T):
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=wtype, dn_wtype=dn_type, shared=True)
    L, _ = make_layer(shape, 70 + T)
    Lt, keep = tabled(L, seed=T)
    x0 = torch.from_numpy(orc.synth(T * shape.H, 900 + T, 1.0).reshape(T, shape.H)).cuda()
    outs = []
    for lay in (L, Lt):
        f = moe.FusedDecode([lay, lay], T)
        x = x0.clone()
        f(x)
        b = moe.DecodeBuffers(shape, T)
        y = torch.empty_like(x0)
        moe.decode_layer(lay, x0, y, b)
        torch.cuda.synchronize()
        outs.append((bits(x), bits(y), b.topi.cpu().numpy()))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])
    assert np.array_equal(outs[0][2], outs[1][2])
    del keep


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q8_0])
def test_prompt_paths_through_tables(wtype):
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=wtype, shared=True)
    L, _ = make_layer(shape, 77)
    Lt, keep = tabled(L, seed=5)
    C = 200
    x = torch.from_numpy(orc.synth(C * shape.H, 901, 1.0).reshape(C, shape.H)).cuda()
    res = []
    for lay in (L, Lt):
        got = []
        for fn in (moe.prefill_layer_mma, moe.prefill_layer_q8):
            b = moe.PrefillBuffers(shape, C)
            y = torch.empty_like(x)
            fn(lay, x, y, b)
            torch.cuda.synchronize()
            got.append(bits(y))
        res.append(got)
    for a, c in zip(res[0], res[1]):
        assert np.array_equal(a, c)
    del keep


def test_table_refuses_nothing_else():
    """a stride of 0 is the table; any other stride smaller than a matrix is still refused"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True)
    L, _ = make_layer(shape, 78)
    b = moe.DecodeBuffers(shape, 1)
    with pytest.raises(RuntimeError, match="stride"):
        moe.moe_gate_up(L.gu_w, 100, shape.wtype, shape.H, 2 * shape.ff, b.jobs_gu, b.njobs, b.njobs_max, 1, b.xq, b.gu)
