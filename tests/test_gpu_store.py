"""GPU parity of the weight store: synthetic values, both quantizers and both dequantizations are bit-exact with the
oracle; GGUF -> planar -> GGUF is the identity."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sfnx_amd import moe

pytestmark = pytest.mark.gpu


def test_synth_bit_exact():
    n, off = 300_001, 12345
    t = torch.empty(n, dtype=torch.float32, device="cuda")
    moe.synth_normal(t, 77, 0.02, offset=off)
    assert np.array_equal(t.cpu().numpy().view(np.uint32), orc.synth(n, 77, 0.02, offset=off).view(np.uint32))


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q5_K, orc.Q4_0, orc.Q5_1, orc.Q8_0])
@pytest.mark.parametrize("rows, cols", [(64, 512), (48, 2048)])
def test_quantizer_bit_exact(wtype, rows, cols):
    x = orc.synth(rows * cols, 5 + cols, 0.02).reshape(rows, cols)
    x[3, :256] = 0.0                      # an all-zero super-block
    x[4, :32] = np.abs(x[4, :32]) + 0.01  # a positive-only sub-block (min clamped to 0)
    xd = torch.from_numpy(x).cuda()
    g = torch.empty(rows * orc.row_bytes(wtype, cols), dtype=torch.uint8, device="cuda")
    moe.quantize_weights(wtype, xd, g)
    assert np.array_equal(g.cpu().numpy(), orc.quantize(wtype, x))


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q5_K, orc.Q4_0, orc.Q5_1, orc.Q8_0])
def test_pack_round_trip_and_dequant(wtype):
    n_mat, rows, cols = 3, 96, 1024
    x = orc.synth(n_mat * rows * cols, 91, 0.02).reshape(n_mat * rows, cols)
    gg = orc.quantize(wtype, x)
    g = torch.from_numpy(gg).cuda()
    planar = torch.empty_like(g)
    back = torch.empty_like(g)
    moe.store_pack(wtype, g, planar, n_mat, rows, cols)
    moe.store_unpack(wtype, planar, back, n_mat, rows, cols)
    assert np.array_equal(back.cpu().numpy(), gg)
    assert not np.array_equal(planar.cpu().numpy(), gg)   # the layout did change
    y = torch.empty((n_mat * rows, cols), dtype=torch.float32, device="cuda")
    moe.dequantize(wtype, planar, y, n_mat, rows, cols)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), orc.dequant(wtype, gg, n_mat * rows, cols).view(np.uint32))
    y16 = torch.empty((n_mat * rows, cols), dtype=torch.float16, device="cuda")
    moe.dequantize_f16(wtype, planar, y16, n_mat, rows, cols)
    assert np.array_equal(y16.cpu().numpy().view(np.uint16), orc.dequant_f16(wtype, gg, n_mat * rows, cols))
