"""The shared expert as its own dense Q8_0 matrices (the reference's Q8S, src/model.hpp:71-83: split int8 and f16-scale
planes) in the reference's q8s arithmetic (src/dense.cuh:24-154): sfnx_q8s_gemv and sfnx_swiglu_stacked_q8_1 against the oracle bit for bit; the
unfused layer against the oracle (gate|up bit-exact, down and the layer within 2e-3 max relative error, as every
layer test: silu uses the device's expf); the fused decode (sfnx_moe_decode_q8s) against the unfused chain bit for
bit; the prompt paths' shared rows (f16 products of the dequantized rows, as the reference's pf_dense_xh) against
float64 within 2e-3."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sfnx_amd import moe
from tests.gpu_util import job_array, make_layer, max_rel

pytestmark = pytest.mark.gpu
TOL = 2e-3


def bits(a):
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else a
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def q8_0_matrix(rows, cols, seed, std=0.02):
    t = torch.from_numpy(orc.synth(rows * cols, seed, std)).cuda()
    g = torch.empty(rows * orc.row_bytes(orc.Q8_0, cols), dtype=torch.uint8, device="cuda")
    moe.quantize_weights(orc.Q8_0, t.view(rows, cols), g)
    return g.cpu().numpy().reshape(rows, -1), moe.Q8sMatrix.from_gguf(g, rows, cols)


@pytest.mark.parametrize("rows,cols", [(32, 512), (96, 2048), (2048, 1024)])
def test_q8s_split_planes(rows, cols):
    """sfnx_q8s_split (src/model.cpp:384-440 q8split): the int8 plane holds each block's 32 values in row order, the
    scale plane each block's f16 bits, [rows][cols / 32]; and the planes give the blocks back"""
    g, W = q8_0_matrix(rows, cols, 17 + rows)
    torch.cuda.synchronize()
    blk = g.reshape(rows, cols // 32, 34)
    assert np.array_equal(W.q.cpu().numpy().view(np.uint8), blk[:, :, 2:].reshape(rows, cols))
    assert np.array_equal(W.d.cpu().numpy().view(np.uint16), blk[:, :, :2].copy().view(np.uint16).reshape(rows, cols // 32))
    assert np.array_equal(W.to_gguf().cpu().numpy(), g.reshape(-1))


@pytest.mark.parametrize("cols", [512, 2048, 4096])
@pytest.mark.parametrize("T", [1, 5, 16])
def test_q8s_gemv_bit_exact(cols, T):
    rows = 96
    g, W = q8_0_matrix(rows, cols, 40 + cols + T)
    x = torch.from_numpy(orc.synth(T * cols, 41 + T, 1.0).reshape(T, cols)).cuda()
    xq = torch.empty(T * cols // 32 * 36, dtype=torch.uint8, device="cuda")
    moe.quantize_q8_1(x, xq)
    stride = rows + 32   # rows of out further apart than the matrix's rows
    out = torch.full((T, stride), 7.0, dtype=torch.float32, device="cuda")
    moe.q8s_gemv(W, rows, cols, xq, out, stride, T)
    torch.cuda.synchronize()
    yq = xq.cpu().numpy().reshape(T, -1)
    want = np.array([[orc.dot_q8s(g[r], yq[t], cols) for r in range(rows)] for t in range(T)], np.float32)
    o = out.cpu().numpy()
    assert np.array_equal(bits(o[:, :rows]), bits(want))
    assert (o[:, rows:] == 7.0).all()
    # and not the routed Q8_0 sums: the two orders differ on some rows
    routed = np.array([orc.dot(orc.Q8_0, g[r], yq[0], cols) for r in range(rows)], np.float32)
    if cols > 512:
        assert (routed != want[0]).any()


@pytest.mark.parametrize("ffs", [512, 1024])
def test_swiglu_stacked_q8_1(ffs):
    T = 7
    gu = orc.synth(T * 2 * ffs, 77, 1.0).reshape(T, 2 * ffs)
    gu[2, :32] = 0.0   # an all-zero block: d = 0, q = 0
    hq = torch.empty(T * ffs // 32 * 36, dtype=torch.uint8, device="cuda")
    moe.swiglu_stacked_q8_1(torch.from_numpy(gu).cuda(), hq, ffs, T)
    torch.cuda.synchronize()
    got = hq.cpu().numpy().reshape(T, -1)
    want = np.stack([orc.swiglu_q8_1(gu[t], ffs) for t in range(T)])
    # silu's expf: the device's and libm's may differ in the last bit, moving a q by one now and then
    blk = got.reshape(T, ffs // 32, 36)
    wblk = want.reshape(T, ffs // 32, 36)
    qd = np.abs(blk[..., 4:].view(np.int8).astype(int) - wblk[..., 4:].view(np.int8).astype(int))
    assert qd.max() <= 1 and np.mean(qd == 0) > 0.999
    d = blk[..., :2].copy().view(np.float16).astype(np.float32)
    wd = wblk[..., :2].copy().view(np.float16).astype(np.float32)
    assert np.allclose(d, wd, rtol=2e-3, atol=0)
    assert (blk[2, 0] == 0).all()


@pytest.mark.parametrize("ffs, T", [(512, 1), (512, 16), (1024, 5)])
def test_q8s_swiglu_gemv_equals_two_calls(ffs, T):
    """the shared expert's SwiGLU and down in one launch (the reference's moe_gate_up sh_down arguments) equals
    swiglu_stacked_q8_1 followed by q8s_gemv, bit for bit"""
    rows = 2048
    _, W = q8_0_matrix(rows, ffs, 90 + ffs + T)
    gu = torch.from_numpy(orc.synth(T * 2 * ffs, 91 + T, 1.0).reshape(T, 2 * ffs)).cuda()
    hq = torch.empty(T * ffs // 32 * 36, dtype=torch.uint8, device="cuda")
    a = torch.full((T, rows), 3.0, dtype=torch.float32, device="cuda")
    b = torch.full((T, rows), 5.0, dtype=torch.float32, device="cuda")
    moe.swiglu_stacked_q8_1(gu, hq, ffs, T)
    moe.q8s_gemv(W, rows, ffs, hq, a, rows, T)
    moe.q8s_swiglu_gemv(W, rows, ffs, gu, b, rows, T)
    torch.cuda.synchronize()
    assert np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("wtype", [orc.Q4_K, orc.Q8_0, orc.Q4_0])
@pytest.mark.parametrize("T", [1, 3, 16])
def test_unfused_layer_q8s_vs_oracle(wtype, T):
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=wtype, shared=True, sh_q8s=True)
    L, host = make_layer(shape, 90 + T + wtype)
    assert L.gu_w.numel() == shape.E * L.gu_stride   # the routed store holds no shared expert
    x = orc.synth(T * shape.H, 910 + T, 1.0).reshape(T, shape.H)
    y = torch.empty((T, shape.H), dtype=torch.float32, device="cuda")
    b = moe.DecodeBuffers(shape, T)
    moe.decode_layer(L, torch.from_numpy(x).cuda(), y, b)
    torch.cuda.synchronize()
    oy, ol, oi, ow, ogu, opart = orc.layer_decode(host, x)
    P = T * shape.K
    assert np.array_equal(b.topi.cpu().numpy(), oi)
    assert int(b.njobs[0]) == len(set(oi[oi >= 0].tolist()))   # no shared job among the routed ones
    sh = list(range(P, P + T))
    assert np.array_equal(bits(b.gu[sh]), bits(ogu[sh])), "shared gate|up not bit-exact"
    # the down dot itself, bit for bit, from the kernel's own h
    hq = b.sh_hq.cpu().numpy().reshape(T, -1)
    dn = host.sh_dn.reshape(shape.H, -1)
    part = b.part.cpu().numpy()
    for t in range(T):
        rows = range(0, shape.H, 37)
        want = np.array([orc.dot_q8s(dn[r], hq[t], shape.ff) for r in rows], np.float32)
        assert np.array_equal(bits(part[P + t, list(rows)]), bits(want))
    assert max_rel(part[sh], opart[sh]) < TOL
    assert max_rel(y.cpu().numpy(), oy) < TOL


@pytest.mark.parametrize("wtype,H", [(orc.Q4_K, 1024), (orc.Q8_0, 1024), (orc.Q5_1, 1024), (orc.Q4_K, 4096),
                                     (orc.Q8_0, 4096)])
@pytest.mark.parametrize("T", [1, 3, 16])
def test_fused_q8s_equals_unfused(wtype, H, T):
    shape = moe.LayerShape(H=H, E=64, K=6, ff=512, wtype=wtype, shared=True, sh_q8s=True)
    layers = [make_layer(shape, 120 + i + T)[0] for i in range(2)]
    x0 = torch.from_numpy(orc.synth(T * H, 930 + T, 1.0).reshape(T, H)).cuda()
    xu = x0.clone()
    xn = torch.empty_like(xu)
    yu = torch.empty_like(xu)
    for L in layers:
        moe.residual_rmsnorm(xu, None, xn)
        b = moe.DecodeBuffers(shape, T)
        moe.decode_layer(L, xn, yu, b)
        xu.add_(yu)
    f = moe.FusedDecode(layers, T)
    xf = x0.clone()
    f(xf, norm=True)
    torch.cuda.synchronize()
    P = T * shape.K
    gf = f.piece("gu", torch.float32, (P + T, 2 * shape.ff))
    assert np.array_equal(bits(gf[P:]), bits(b.gu[P:P + T]))
    assert np.array_equal(bits(f.piece("y", torch.float32, (T, H))), bits(yu))
    assert np.array_equal(bits(xf), bits(xu))


def test_fused_q8s_baseline_shape():
    """the benchmark layer shape (hidden 2048, 512 experts x FF 512, top-10) with a dense Q8_0 shared expert"""
    shape = moe.LayerShape(H=2048, E=512, K=10, ff=512, wtype=orc.Q4_K, shared=True, sh_q8s=True)
    L, host = make_layer(shape, 5)
    for T in (1, 16):
        x = orc.synth(T * shape.H, 940 + T, 1.0).reshape(T, shape.H)
        xf = torch.from_numpy(x).cuda()
        f = moe.FusedDecode([L], T)
        f(xf, norm=False)
        torch.cuda.synchronize()
        oy, ol, oi, ow, ogu, opart = orc.layer_decode(host, x, nthreads=8)
        P = T * shape.K
        gf = f.piece("gu", torch.float32, (P + T, 2 * shape.ff)).cpu().numpy()
        assert np.array_equal(bits(gf[P:]), bits(ogu[P:]))
        assert max_rel(f.piece("y", torch.float32, (T, shape.H)).cpu().numpy(), oy) < TOL


def shared_rows_f64(host, x, C):
    """float64 shared expert rows P + t of the f16 prompt path: f16 weights (d q, rounded), f16 x, f16 h"""
    s = host
    gw = orc.dequant(orc.Q8_0, host.sh_gu, 2 * s.ff, s.H).astype(np.float16).astype(np.float64)
    dw = orc.dequant(orc.Q8_0, host.sh_dn, s.H, s.ff).astype(np.float16).astype(np.float64)
    g = x.astype(np.float16).astype(np.float64) @ gw.T
    h = (g[:, : s.ff] / (1 + np.exp(-g[:, : s.ff])) * g[:, s.ff:]).astype(np.float16).astype(np.float64)
    return h @ dw.T


@pytest.mark.parametrize("path", ["mma", "q8"])
def test_prefill_shared_q8s(path):
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True, sh_q8s=True)
    L, host = make_layer(shape, 150)
    C = 150
    x = orc.synth(C * shape.H, 960, 1.0).reshape(C, shape.H)
    xd = torch.from_numpy(x).cuda()
    y = torch.empty_like(xd)
    b = moe.PrefillBuffers(shape, C)
    if path == "mma":
        moe.prefill_layer_mma(L, xd, y, b)
    else:
        moe.prefill_layer_q8(L, xd, y, b)
    torch.cuda.synchronize()
    P = C * shape.K
    jobs = job_array(b.jobs_gu, True)[: int(b.njobs[0])]
    assert (jobs["w"] < shape.E).all()   # the routed jobs only
    want = shared_rows_f64(host, x, C)
    got = b.part.cpu().numpy()[P:P + C]
    assert max_rel(got, want) < TOL
    # the layer: the combine of the kernel's own rows
    topi, topw = b.topi.cpu().numpy(), b.topw.cpu().numpy().astype(np.float64)
    part = b.part.cpu().numpy().astype(np.float64)
    sig = 1 / (1 + np.exp(-b.logits.cpu().numpy()[:, shape.E].astype(np.float64)))
    ref = np.einsum("tk,tkh->th", topw, part[:P].reshape(C, shape.K, -1)) + sig[:, None] * part[P:]
    assert max_rel(y.cpu().numpy(), ref) < 1e-5


def test_synthetic_q8s_layer():
    """MoeLayer.synthetic with a dense shared expert: its matrices are expert E of a Q8_0 layer of the same seed, the
    routed experts those of the Q4_K layer, and a decode step is finite and equal to the oracle's"""
    s = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True, sh_q8s=True)
    L = moe.MoeLayer.synthetic(s, seed=31)
    R = moe.MoeLayer.synthetic(moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q8_0, shared=True), seed=31)
    Q = moe.MoeLayer.synthetic(moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True), seed=31)
    assert L.W.shape == (s.E + 1, s.H) and torch.equal(L.W, Q.W)
    rg, rd = torch.empty(R.gu_stride, dtype=torch.uint8, device="cuda"), torch.empty(R.dn_stride, dtype=torch.uint8, device="cuda")
    moe.store_unpack(orc.Q8_0, R.gu_w[s.E * R.gu_stride:(s.E + 1) * R.gu_stride], rg, 1, 2 * s.ff, s.H)
    moe.store_unpack(orc.Q8_0, R.dn_w[s.E * R.dn_stride:(s.E + 1) * R.dn_stride], rd, 1, s.H, s.ff)
    assert torch.equal(L.sh_gu.to_gguf(), rg) and torch.equal(L.sh_dn.to_gguf(), rd)
    assert torch.equal(L.gu_w, Q.gu_w[: s.E * Q.gu_stride]) and torch.equal(L.dn_w, Q.dn_w[: s.E * Q.dn_stride])
    x = orc.synth(s.H, 990, 1.0).reshape(1, s.H)
    f = moe.FusedDecode([L], 1)
    xf = torch.from_numpy(x).cuda()
    f(xf, norm=False)
    torch.cuda.synchronize()
    gu = torch.empty_like(L.gu_w)
    dn = torch.empty_like(L.dn_w)
    moe.store_unpack(orc.Q4_K, L.gu_w, gu, s.E, 2 * s.ff, s.H)
    moe.store_unpack(orc.Q4_K, L.dn_w, dn, s.E, s.H, s.ff)
    sg, sd = L.sh_gu.to_gguf(), L.sh_dn.to_gguf()
    host = orc.LayerWeights(L.W.cpu().numpy(), gu.cpu().numpy(), dn.cpu().numpy(), s.wtype, s.H, s.E, s.K, s.ff, True,
                            sh_gu=sg.cpu().numpy(), sh_dn=sd.cpu().numpy())
    oy = orc.layer_decode(host, x)[0]
    yf = f.piece("y", torch.float32, (1, s.H)).cpu().numpy()
    assert np.isfinite(yf).all() and max_rel(yf, oy) < TOL


@pytest.mark.parametrize("rows,cols,C", [(1024, 2048, 200), (2048, 512, 33), (512, 1024, 1000), (256, 512, 1)])
def test_pf_dense_against_float64(rows, cols, C):
    """sfnx_pf_dense (src/prefill.cu:407-417): f16(W) . xh rows in fp32, against float64 products of the same f16
    operands within 2e-3 (the sum's order is the matrix-core kernel's, as the reference's is cuBLAS's); rows of out
    ldo apart, the columns past rows untouched"""
    g, W = q8_0_matrix(rows, cols, 300 + cols)
    x = orc.synth(C * cols, 301, 1.0).reshape(C, cols).astype(np.float16)
    ldo = rows + 64
    out = torch.full((C, ldo), 5.0, dtype=torch.float32, device="cuda")
    wh = torch.empty(rows * cols, dtype=torch.float16, device="cuda")
    moe.pf_dense(W, rows, cols, torch.from_numpy(x).cuda(), out, ldo, wh)
    torch.cuda.synchronize()
    w16 = orc.dequant(orc.Q8_0, g.reshape(-1), rows, cols).astype(np.float16).astype(np.float64)
    want = x.astype(np.float64) @ w16.T
    got = out.cpu().numpy()
    assert max_rel(got[:, :rows], want) < 2e-3
    assert (got[:, rows:] == 5.0).all()


def test_pf_dense_refuses_a_small_staging_buffer():
    _, W = q8_0_matrix(256, 512, 5)
    xh = torch.zeros((4, 512), dtype=torch.float16, device="cuda")
    out = torch.empty((4, 256), dtype=torch.float32, device="cuda")
    wh = torch.empty(256 * 512 // 2, dtype=torch.float16, device="cuda")   # 256 KB, below 256 * 512 * 34 / 32 bytes
    with pytest.raises(RuntimeError, match="wk smaller"):
        moe.pf_dense(W, 256, 512, xh, out, 256, wh)


def test_prefill_shared_graph_replays():
    """the dense shared expert's prompt rows (job lists + matrix-core GEMMs) captured in a HIP graph, as the bench
    times them: every replay, with eager work between them, equals the eager result bit for bit"""
    shape = moe.LayerShape(H=1024, E=64, K=6, ff=512, wtype=orc.Q4_K, shared=True, sh_q8s=True)
    L, _ = make_layer(shape, 160)
    C = 96
    P = C * shape.K
    b = moe.PrefillBuffers(shape, C)
    moe.to_f16(torch.from_numpy(orc.synth(C * shape.H, 161, 1.0).reshape(C, shape.H)).cuda(), b.xh)
    moe.prefill_shared(L, b)
    torch.cuda.synchronize()
    want = b.part[P:P + C].clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        moe.prefill_shared(L, b)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        moe.prefill_shared(L, b)
    for i in range(3):
        b.part[P:P + C].fill_(float(i + 1))   # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(b.part[P:P + C], want), i
