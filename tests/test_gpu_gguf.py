"""A MoE layer loaded from a GGUF file into the device store (sfnx_gguf_moe_layer; src/model.cpp:554-606 and 766-809)
against the bytes the test wrote: the store unpacked to GGUF layout equals the sliced source tensors byte for byte,
the router equals [ffn_gate_inp ; ffn_gate_inp_shexp], and one decode window through the loaded layer equals the oracle
on the same bytes (top-k indices bit-exact, outputs within 2e-3 max relative error)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sfnx_amd import moe
from tests import gguf_writer as gw
from tests.gpu_util import max_rel

pytestmark = pytest.mark.gpu


def _layer_bytes(wtype, H, E, ff, seed, dn_type=None, sh_type=None):
    rng = np.random.default_rng(seed)
    dt = wtype if dn_type is None else dn_type
    q = lambda r, c, t=wtype: orc.quantize(t, (0.02 * rng.standard_normal((r, c))).astype(np.float32))
    gate = np.stack([q(ff, H) for _ in range(E)])
    up = np.stack([q(ff, H) for _ in range(E)])
    down = np.stack([q(H, ff, dt) for _ in range(E)])
    st = sh_type or wtype
    shared = (q(ff, H, st), q(ff, H, st), q(H, ff, sh_type or dt), (0.02 * rng.standard_normal(H)).astype(np.float32))
    W = (0.02 * rng.standard_normal((E, H))).astype(np.float32)
    return W, gate, up, down, shared


@pytest.mark.parametrize("wtype,dn,H,E,ff,ff0,ff1", [
    (orc.Q4_K, None, 1024, 64, 512, 0, 512), (orc.Q4_K, None, 1024, 64, 1024, 256, 768),
    (orc.Q5_K, None, 1024, 64, 1024, 256, 768), (orc.Q4_0, None, 1024, 64, 512, 0, 512),
    (orc.Q5_1, None, 1024, 64, 1024, 32, 544), (orc.Q8_0, None, 1024, 64, 512, 0, 512),
    (orc.Q8_0, None, 1024, 64, 1024, 32, 544),
    # gate and up in one type, down in another (src/model.cpp:540-606)
    (orc.Q4_K, orc.Q5_K, 1024, 64, 1024, 256, 768), (orc.Q4_K, orc.Q8_0, 1024, 64, 512, 0, 512)])
def test_gguf_layer(tmp_path, wtype, dn, H, E, ff, ff0, ff1):
    W, gate, up, down, shared = _layer_bytes(wtype, H, E, ff, 11, dn)
    dty = wtype if dn is None else dn
    path = tmp_path / "layer.gguf"
    gw.write_gguf(path, [("general.architecture", gw.STR, "qwen3moe")],
                  gw.moe_layer_tensors(3, W, gate, up, down, wtype, H, E, ff, shared, dn))
    g = moe.Gguf(str(path))
    L = moe.gguf_moe_layer(g, 3, ff0, ff1, K=4)
    torch.cuda.synchronize()
    s = L.s
    ffs = ff1 - ff0
    assert s.shared and s.E == E and s.H == H and s.ff == ffs and s.wtype == wtype and s.dn_type == dty
    # the router: routed rows, then the shared gate row
    assert np.array_equal(L.W.cpu().numpy(), np.vstack([W, shared[3][None]]))
    # the store, unpacked to GGUF layout, against the sliced source bytes
    rb_h, rb_f, rb_full = orc.row_bytes(wtype, H), orc.row_bytes(dty, ffs), orc.row_bytes(dty, ff)
    col0 = orc.row_bytes(dty, ff0)
    gu_g = torch.empty_like(L.gu_w)
    dn_g = torch.empty_like(L.dn_w)
    moe.store_unpack(wtype, L.gu_w, gu_g, E + 1, 2 * ffs, H)
    moe.store_unpack(dty, L.dn_w, dn_g, E + 1, H, ffs)
    gu_h = gu_g.cpu().numpy().reshape(E + 1, 2 * ffs, rb_h)
    dn_h = dn_g.cpu().numpy().reshape(E + 1, H, rb_f)
    for e in range(E + 1):
        gt, ut, dt = (shared[0], shared[1], shared[2]) if e == E else (gate[e], up[e], down[e])
        assert np.array_equal(gu_h[e, :ffs], gt.reshape(ff, rb_h)[ff0:ff1])
        assert np.array_equal(gu_h[e, ffs:], ut.reshape(ff, rb_h)[ff0:ff1])
        assert np.array_equal(dn_h[e], dt.reshape(H, rb_full)[:, col0:col0 + rb_f])
    # one decode window through the loaded layer against the oracle on the same bytes
    host = orc.LayerWeights(L.W.cpu().numpy(), gu_h.reshape(-1), dn_h.reshape(-1), wtype, H, E, s.K, ffs, True, dn_type=dty)
    T = 3
    x = orc.synth(T * H, 77, 1.0).reshape(T, H)
    y = torch.empty((T, H), dtype=torch.float32, device="cuda")
    b = moe.DecodeBuffers(s, T)
    moe.decode_layer(L, torch.from_numpy(x).cuda(), y, b)
    torch.cuda.synchronize()
    oy, _, oi, _, _, _ = orc.layer_decode(host, x)
    assert np.array_equal(b.topi.cpu().numpy(), oi)
    assert max_rel(y.cpu().numpy(), oy) < 2e-3


def test_gguf_layer_refusals(tmp_path):
    W, gate, up, down, shared = _layer_bytes(orc.Q4_K, 512, 64, 512, 12)
    path = tmp_path / "l.gguf"
    gw.write_gguf(path, [], gw.moe_layer_tensors(0, W, gate, up, down, orc.Q4_K, 512, 64, 512, shared))
    g = moe.Gguf(str(path))
    with pytest.raises(RuntimeError, match="missing"):
        moe.gguf_moe_layer(g, 1)
    with pytest.raises(RuntimeError, match="whole block"):
        moe.gguf_moe_layer(g, 0, 128, 512)
    # the caller's buffers against the file's E (64 routed + the shared expert): one expert short of each is refused
    # before anything is written
    H, E, ff = 512, 64, 512
    gs, ds = 2 * ff * orc.row_bytes(orc.Q4_K, H), H * orc.row_bytes(orc.Q4_K, ff)
    gu = torch.full(((E + 1) * gs,), 7, dtype=torch.uint8, device="cuda")
    dn = torch.full(((E + 1) * ds,), 7, dtype=torch.uint8, device="cuda")
    Wt = torch.zeros((E + 1, H), dtype=torch.float32, device="cuda")
    lib, p = moe.lib(), moe._p
    for gb, db, wr, msg in [(E * gs, (E + 1) * ds, E + 1, "gu buffer too small"), ((E + 1) * gs, E * ds, E + 1, "dn buffer too small"),
                            ((E + 1) * gs, (E + 1) * ds, E, "router rows")]:
        assert lib.sfnx_gguf_moe_layer(g._h, 0, 0, ff, p(gu), gs, gb, p(dn), ds, db, p(Wt), wr, None, None) == -1
        assert msg in lib.sfnx_last_error().decode()
    torch.cuda.synchronize()
    assert (gu == 7).all() and (dn == 7).all()
    assert lib.sfnx_gguf_moe_layer(g._h, 0, 0, ff, p(gu), gs, gu.numel(), p(dn), ds, dn.numel(), p(Wt), E + 1, None, None) == 0


@pytest.mark.parametrize("wtype,ff,ff0,ff1", [(orc.Q4_K, 512, 0, 512), (orc.Q4_K, 1024, 256, 768), (orc.Q5_1, 1024, 32, 544)])
def test_gguf_layer_q8s_shared(tmp_path, wtype, ff, ff0, ff1):
    """the shared expert as the reference loads it (src/model.cpp:807-809): Q8_0 in the file, dense matrices on the
    device; the routed stores hold E experts; decode (unfused and fused) against the oracle on the same bytes"""
    H, E = 1024, 64
    W, gate, up, down, shared = _layer_bytes(wtype, H, E, ff, 13, sh_type=orc.Q8_0)
    path = tmp_path / "layer.gguf"
    gw.write_gguf(path, [], gw.moe_layer_tensors(2, W, gate, up, down, wtype, H, E, ff, shared, sh_type=orc.Q8_0))
    g = moe.Gguf(str(path))
    L = moe.gguf_moe_layer(g, 2, ff0, ff1, K=4, q8s=True)
    torch.cuda.synchronize()
    s = L.s
    ffs = ff1 - ff0
    assert s.sh_q8s and s.shared and L.gu_w.numel() == E * L.gu_stride
    rb_h, rb_f, rb_full = orc.row_bytes(orc.Q8_0, H), orc.row_bytes(orc.Q8_0, ffs), orc.row_bytes(orc.Q8_0, ff)
    col0 = orc.row_bytes(orc.Q8_0, ff0)
    sg, sd = L.sh_gu.to_gguf().cpu().numpy(), L.sh_dn.to_gguf().cpu().numpy()
    want_g = np.concatenate([shared[0].reshape(ff, rb_h)[ff0:ff1], shared[1].reshape(ff, rb_h)[ff0:ff1]])
    assert np.array_equal(sg.reshape(2 * ffs, rb_h), want_g)
    assert np.array_equal(sd.reshape(H, rb_f), shared[2].reshape(H, rb_full)[:, col0:col0 + rb_f])
    # routed stores unpacked for the oracle
    gu_g = torch.empty_like(L.gu_w)
    dn_g = torch.empty_like(L.dn_w)
    moe.store_unpack(wtype, L.gu_w, gu_g, E, 2 * ffs, H)
    moe.store_unpack(wtype, L.dn_w, dn_g, E, H, ffs)
    host = orc.LayerWeights(L.W.cpu().numpy(), gu_g.cpu().numpy(), dn_g.cpu().numpy(), wtype, H, E, s.K, ffs, True,
                            sh_gu=sg, sh_dn=sd)
    T = 3
    x = orc.synth(T * H, 78, 1.0).reshape(T, H)
    y = torch.empty((T, H), dtype=torch.float32, device="cuda")
    b = moe.DecodeBuffers(s, T)
    moe.decode_layer(L, torch.from_numpy(x).cuda(), y, b)
    xf = torch.from_numpy(x).cuda()
    moe.FusedDecode([L], T)(xf, norm=False)
    torch.cuda.synchronize()
    oy, _, oi, _, ogu, _ = orc.layer_decode(host, x)
    assert np.array_equal(b.topi.cpu().numpy(), oi)
    P = T * s.K
    assert np.array_equal(b.gu.cpu().numpy()[P:].view(np.uint32), ogu[P:].view(np.uint32))
    assert max_rel(y.cpu().numpy(), oy) < 2e-3
    # the fused decode: x + y of the unfused layer, bit for bit
    assert np.array_equal(xf.cpu().numpy().view(np.uint32), (torch.from_numpy(x).cuda() + y).cpu().numpy().view(np.uint32))
    # a shared expert of another type is refused on this path, as the reference refuses it
    path2 = tmp_path / "l2.gguf"
    W2, g2, u2, d2, sh2 = _layer_bytes(wtype, H, E, ff, 14)
    gw.write_gguf(path2, [], gw.moe_layer_tensors(0, W2, g2, u2, d2, wtype, H, E, ff, sh2))
    with pytest.raises(RuntimeError, match="not Q8_0"):
        moe.gguf_moe_layer(moe.Gguf(str(path2)), 0, q8s=True)
