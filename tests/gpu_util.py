"""Helpers for the GPU parity tests: seeded layers built on the device (synthetic values, the library's quantizer,
the planar store) with the same GGUF bytes copied to the host for the oracle."""
import numpy as np
import torch

from oracle import oracle as orc
from sfnx_amd import moe


def job_array(t: torch.Tensor, big: bool = False) -> np.ndarray:
    dt = orc.BIGJOB_DTYPE if big else orc.JOB_DTYPE
    return t.cpu().numpy().view(dt)


def make_layer(shape: moe.LayerShape, seed: int, device="cuda"):
    """(device MoeLayer, oracle LayerWeights) holding the same weights"""
    s = shape
    E1 = s.E + 1
    gu_stride = 2 * s.ff * moe.row_bytes(s.wtype, s.H)
    dn_stride = s.H * moe.row_bytes(s.dn_type, s.ff)
    W = torch.empty((E1, s.H), dtype=torch.float32, device=device)
    moe.synth_normal(W, seed * 1000 + 1, 0.02)
    gu_g = torch.empty(E1 * gu_stride, dtype=torch.uint8, device=device)
    dn_g = torch.empty(E1 * dn_stride, dtype=torch.uint8, device=device)
    for rows, cols, dst, sd, wt in ((E1 * 2 * s.ff, s.H, gu_g, seed * 1000 + 2, s.wtype),
                                    (E1 * s.H, s.ff, dn_g, seed * 1000 + 3, s.dn_type)):
        chunk = 1 << 24
        total = rows * cols
        per = max(cols, chunk // cols * cols)
        tmp = torch.empty(per, dtype=torch.float32, device=device)
        rb = moe.row_bytes(wt, cols)
        for off in range(0, total, per):
            n = min(per, total - off)
            moe.synth_normal(tmp[:n], sd, 0.02, offset=off)
            r0 = off // cols
            moe.quantize_weights(wt, tmp[:n].view(n // cols, cols), dst[r0 * rb:(r0 + n // cols) * rb])
    sh = [None, None]
    if s.sh_q8s:   # the shared expert as dense Q8_0: expert E's values of the same streams
        for i, (rows, cols, sd) in enumerate(((2 * s.ff, s.H, seed * 1000 + 2), (s.H, s.ff, seed * 1000 + 3))):
            tmp = torch.empty(rows * cols, dtype=torch.float32, device=device)
            moe.synth_normal(tmp, sd, 0.02, offset=s.E * rows * cols)
            sh[i] = torch.empty(rows * moe.row_bytes(orc.Q8_0, cols), dtype=torch.uint8, device=device)
            moe.quantize_weights(orc.Q8_0, tmp.view(rows, cols), sh[i])
        # the routed stores hold E experts: nothing may read an expert E
        L = moe.MoeLayer.planar_from_gguf(s, W, gu_g[: s.E * gu_stride], dn_g[: s.E * dn_stride], sh[0], sh[1])
    else:
        L = moe.MoeLayer.planar_from_gguf(s, W, gu_g, dn_g)
    torch.cuda.synchronize()
    host = orc.LayerWeights(W.cpu().numpy(), gu_g.cpu().numpy(), dn_g.cpu().numpy(), s.wtype, s.H, s.E, s.K, s.ff,
                            s.shared, dn_type=s.dn_type, sh_gu=None if sh[0] is None else sh[0].cpu().numpy(),
                            sh_dn=None if sh[1] is None else sh[1].cpu().numpy())
    return L, host


def max_rel(got, want) -> float:
    """max |got - want| over max |want| (the tolerance measure of tools/moe_mma_bench.cu:197-220)"""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def tabled(L: moe.MoeLayer, seed: int = 0):
    """the same layer with its experts moved and reached through device pointer tables (stride 0; the reference's
    DW::ep): each expert's matrices copied to a new, shuffled place in one fresh buffer, the tables pointing there.
    Returns (layer view, the buffers it holds) - keep the buffers alive while the view is used."""
    import copy
    s = L.s
    n = L.gu_w.numel() // L.gu_stride
    perm = np.random.default_rng(seed).permutation(n)
    keep = []
    view = copy.copy(L)
    for name, stride in (("gu_w", L.gu_stride), ("dn_w", L.dn_stride)):
        src = getattr(L, name)
        pitch = (stride + 255) // 256 * 256 + 256   # gaps between the moved matrices
        dst = torch.full((n * pitch,), 0xEE, dtype=torch.uint8, device=src.device)
        for e in range(n):
            dst[perm[e] * pitch: perm[e] * pitch + stride].copy_(src[e * stride:(e + 1) * stride])
        table = torch.tensor([dst.data_ptr() + int(perm[e]) * pitch for e in range(n)], dtype=torch.int64,
                             device=src.device)
        keep += [dst, table]
        setattr(view, name, table)
        setattr(view, name.replace("_w", "_stride"), 0)
    return view, keep
