"""Python host mirror of the reference engine's MoE entry points (src/kernels.hpp:269-313) over the C ABI.

torch supplies device memory and the current stream; every computation is a call into libsfnx_moe.so.  Functions keep
the reference's names and argument meaning; shapes that the reference fixes at compile time (N, NEXP, TOPK) are
arguments here.  Errors from the library raise RuntimeError, as the reference's wrappers throw (src/kernels.cu:31-34).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _abi
from ._abi import BIGJOB_INTS, JOB_INTS, PF_JOB, Q4_0, Q4_K, Q5_1, Q5_K, Q8_0, check, lib


def _p(t):
    return None if t is None else t.data_ptr()


def _st():
    return torch.cuda.current_stream().cuda_stream


def row_bytes(wtype: int, cols: int) -> int:
    return lib().sfnx_row_bytes(wtype, cols)


# ---------------------------------------------------------------------------------------------------- store
def synth_normal(out: torch.Tensor, seed: int, std: float, offset: int = 0) -> None:
    check(lib().sfnx_synth_normal(_p(out), out.numel(), seed, offset, std, _st()))


def quantize_weights(wtype: int, x: torch.Tensor, gguf: torch.Tensor) -> None:
    rows, cols = x.shape
    check(lib().sfnx_quantize_weights(wtype, _p(x), _p(gguf), rows, cols, _st()))


def store_pack(wtype: int, gguf: torch.Tensor, planar: torch.Tensor, n_mat: int, rows: int, cols: int) -> None:
    check(lib().sfnx_store_pack(wtype, _p(gguf), _p(planar), n_mat, rows, cols, _st()))


def store_unpack(wtype: int, planar: torch.Tensor, gguf: torch.Tensor, n_mat: int, rows: int, cols: int) -> None:
    check(lib().sfnx_store_unpack(wtype, _p(planar), _p(gguf), n_mat, rows, cols, _st()))


def dequantize(wtype: int, planar: torch.Tensor, y: torch.Tensor, n_mat: int, rows: int, cols: int) -> None:
    check(lib().sfnx_dequantize(wtype, _p(planar), _p(y), n_mat, rows, cols, _st()))


def dequantize_f16(wtype: int, planar: torch.Tensor, y: torch.Tensor, n_mat: int, rows: int, cols: int) -> None:
    check(lib().sfnx_dequantize_f16(wtype, _p(planar), _p(y), n_mat, rows, cols, _st()))


# ---------------------------------------------------------------------------------------------------- routing
def quantize_q8_1(x: torch.Tensor, q: torch.Tensor) -> None:
    rows, n = x.shape
    check(lib().sfnx_quantize_q8_1(_p(x), _p(q), n, rows, _st()))


def router_route(W, x, logits, topi, topw, jobs_gu, jobs_dn, njobs, E: int, K: int, shared: bool = True,
                 plan=None) -> None:
    """src/kernels.hpp:269-278 router_route; plan = (cache, layer, list): the same launch's last block also plans the
    window's slots in the ExpertCache (sfnx_router_route_plan)"""
    T, H = x.shape
    if plan is None:
        check(lib().sfnx_router_route(_p(W), _p(x), _p(logits), T, H, E, K, _p(topi), _p(topw), _p(jobs_gu),
                                      _p(jobs_dn), _p(njobs), int(shared), _st()))
    else:
        cache, layer, out_list = plan
        check(lib().sfnx_router_route_plan(_p(W), _p(x), _p(logits), T, H, E, K, _p(topi), _p(topw), _p(jobs_gu),
                                           _p(jobs_dn), _p(njobs), int(shared), C.byref(cache.c), layer, _p(out_list),
                                           _st()))


def router_logits(W, x, logits) -> None:
    T, H = x.shape
    check(lib().sfnx_router_logits(_p(W), _p(x), _p(logits), T, H, W.shape[0], _st()))


def router_logits_xh(W, x, logits, xh) -> None:
    """router_logits and xh = f16(x) from one read of x"""
    T, H = x.shape
    check(lib().sfnx_router_logits_xh(_p(W), _p(x), _p(logits), _p(xh), T, H, W.shape[0], _st()))


def pf_route(logits, topi, topw, cnt, jbase, jobs_gu, jobs_dn, njobs, E: int, K: int, shared: bool = True) -> None:
    C = logits.shape[0]
    check(lib().sfnx_pf_route(_p(logits), C, E, K, _p(topi), _p(topw), _p(cnt), _p(jbase), _p(jobs_gu), _p(jobs_dn),
                              _p(njobs), int(shared), _st()))


# ---------------------------------------------------------------------------------------------------- experts
def moe_gate_up(A, sa, wtype, n_in, n_out, jobs, njobs, njobs_max, T, xq, gu) -> None:
    check(lib().sfnx_moe_gate_up(_p(A), sa, wtype, n_in, n_out, _p(jobs), _p(njobs), njobs_max, T, _p(xq), _p(gu), _st()))


def moe_down(A, sa, wtype, n_in, n_out, jobs, njobs, njobs_max, T, gu, part) -> None:
    check(lib().sfnx_moe_down(_p(A), sa, wtype, n_in, n_out, _p(jobs), _p(njobs), njobs_max, T, _p(gu), _p(part), _st()))


def moe_gate_up_big(A, sa, wtype, n_in, n_out, jobs, njobs, njobs_cap, xq, gu) -> None:
    check(lib().sfnx_moe_gate_up_big(_p(A), sa, wtype, n_in, n_out, _p(jobs), _p(njobs), njobs_cap, _p(xq), _p(gu), _st()))


def moe_down_big(A, sa, wtype, n_in, n_out, jobs, njobs, njobs_cap, gu, part) -> None:
    check(lib().sfnx_moe_down_big(_p(A), sa, wtype, n_in, n_out, _p(jobs), _p(njobs), njobs_cap, _p(gu), _p(part), _st()))


def moe_gate_up_mma(A, sa, wtype, n_in, n_out, jobs, njobs, njobs_cap, xh, gu) -> None:
    check(lib().sfnx_moe_gate_up_mma(_p(A), sa, wtype, n_in, n_out, _p(jobs), _p(njobs), njobs_cap, _p(xh), _p(gu), _st()))


def swiglu_h16(gu, h16, ff: int) -> None:
    check(lib().sfnx_swiglu_h16(_p(gu), ff, gu.shape[0], _p(h16), _st()))


def moe_gate_up_swiglu_mma(A, sa, wtype, n_in, ff, jobs, njobs, njobs_cap, xh, h16) -> None:
    check(lib().sfnx_moe_gate_up_swiglu_mma(_p(A), sa, wtype, n_in, ff, _p(jobs), _p(njobs), njobs_cap, _p(xh), _p(h16), _st()))


def moe_down_mma(A, sa, wtype, n_in, n_out, jobs, njobs, njobs_cap, h16, part) -> None:
    check(lib().sfnx_moe_down_mma(_p(A), sa, wtype, n_in, n_out, _p(jobs), _p(njobs), njobs_cap, _p(h16), _p(part), _st()))


def to_f16(x, y) -> None:
    check(lib().sfnx_to_f16(_p(x), _p(y), x.numel(), _st()))


def moe_combine(part, topw, topi, logits, y, E: int, K: int, shared: bool = True) -> None:
    T, H = y.shape
    check(lib().sfnx_moe_combine(_p(part), _p(topw), _p(topi), _p(logits), _p(y), T, H, E, K, int(shared), _st()))


class Q8sMatrix:
    """src/model.hpp:71-74 Q8S: a dense Q8_0 matrix [rows][cols] in the reference's split layout (src/model.cpp:384-440
    q8split): int8 values q [rows][cols] and the f16 scale bits d [rows][cols / 32] (held as int16), two allocations.
    `c` is the sfnx_q8s struct the C ABI takes (by address, ptr())."""

    def __init__(self, rows: int, cols: int, device="cuda"):
        self.rows, self.cols = rows, cols
        self.q = torch.empty((rows, cols), dtype=torch.int8, device=device)
        self.d = torch.empty((rows, cols // 32), dtype=torch.int16, device=device)
        self.c = _abi.Q8S(self.q.data_ptr(), self.d.data_ptr())

    def ptr(self) -> int:
        return C.addressof(self.c)

    @staticmethod
    def from_gguf(blocks: torch.Tensor, rows: int, cols: int) -> "Q8sMatrix":
        """GGUF Q8_0 blocks [rows][cols / 32] split on the device (sfnx_q8s_split)"""
        m = Q8sMatrix(rows, cols, device=blocks.device)
        check(lib().sfnx_q8s_split(_p(blocks), rows, cols, m.ptr(), _st()))
        return m

    def to_gguf(self) -> torch.Tensor:
        """the GGUF Q8_0 blocks (uint8 [rows * cols / 32 * 34]) of the matrix"""
        d = self.d.reshape(-1, 1).view(torch.uint8).reshape(-1, 2)
        q = self.q.reshape(-1, 32).view(torch.uint8)
        return torch.cat([d, q], dim=1).reshape(-1)


def q8s_gemv(W: "Q8sMatrix", rows: int, cols: int, y, out, out_stride: int, T: int) -> None:
    """src/kernels.hpp:47: out[t][r] = dense Q8_0 row r of W (split layout) . q8_1 row t of y, the reference's q8s sums
    (src/dense.cuh:24-154); out rows out_stride floats apart"""
    check(lib().sfnx_q8s_gemv(W.ptr(), rows, cols, _p(y), _p(out), out_stride, T, _st()))


def swiglu_stacked_q8_1(gu, hq, ffs: int, T: int) -> None:
    """src/kernels.cu:2018: hq row t (q8_1) = silu(gate) * up of gu row t ([gate | up], 2 ffs floats)"""
    check(lib().sfnx_swiglu_stacked_q8_1(_p(gu), _p(hq), ffs, T, _st()))


def q8s_swiglu_gemv(W, rows: int, ffs: int, gu, out, out_stride: int, T: int) -> None:
    """src/kernels.hpp:281-282's shared-expert tail in one launch: out[t][r] = dense Q8_0 row r of W . q8_1 of
    silu(gate) * up of gu row t ([gate | up], 2 ffs floats); equal to swiglu_stacked_q8_1 then q8s_gemv"""
    check(lib().sfnx_q8s_swiglu_gemv(W.ptr(), rows, ffs, _p(gu), _p(out), out_stride, T, _st()))


def residual_rmsnorm(x, y, xn, eps: float = 1e-6) -> None:
    """x += y (y may be None), xn = x / sqrt(mean(x^2) + eps): the glue between stacked layers"""
    T, H = x.shape
    check(lib().sfnx_residual_rmsnorm(_p(x), _p(y), _p(xn), T, H, eps, _st()))


def kernel_clock(enable: bool) -> None:
    """stamp each decode kernel's own begin/end (a measurement aid; see kernel_clock_read)"""
    check(lib().sfnx_kernel_clock(int(enable)))


def kernel_clock_read() -> list:
    """durations in us of the last clocked decode launches: [router, gate|up, down + combine]"""
    us = (C.c_float * 3)()
    check(lib().sfnx_kernel_clock_read(C.cast(us, C.c_void_p)))
    return list(us)


# ---------------------------------------------------------------------------------------------------- a layer
@dataclass
class LayerShape:
    H: int = 2048
    E: int = 512
    K: int = 10
    ff: int = 512
    wtype: int = Q4_K
    shared: bool = True
    dn_wtype: int | None = None   # the down matrices' type when it differs from gate|up's (the reference's DW per matrix)
    # the shared expert as its own dense Q8_0 matrices in the reference's q8s arithmetic (src/model.hpp:83 DW::s,
    # src/engine.cu:936-945); the routed stores then hold E experts.  Else it is expert E of the routed stores.
    sh_q8s: bool = False

    @property
    def n_routed(self) -> int:
        """experts in the routed stores"""
        return self.E + (0 if self.sh_q8s else 1)

    @property
    def dn_type(self) -> int:
        return self.wtype if self.dn_wtype is None else self.dn_wtype


class MoeLayer:
    """One MoE layer's weights resident in HBM (planar store) plus the buffers its entry points write.

    gu_w: experts' gate|up [E+1][2 ff][H] (expert E is the shared one), dn_w: down [E+1][H][ff], W: router [E+1][H].
    With shape.sh_q8s the stores hold E experts and sh_gu [2 ff][H], sh_dn [H][ff] (Q8sMatrix, the reference's split
    Q8_0 layout) the shared expert.
    """

    def __init__(self, shape: LayerShape, W: torch.Tensor, gu_w: torch.Tensor, dn_w: torch.Tensor,
                 sh_gu: "Q8sMatrix | None" = None, sh_dn: "Q8sMatrix | None" = None):
        if W.shape[0] != shape.E + 1:
            raise ValueError("the router has E + 1 rows (row E gates the shared expert)")
        if shape.sh_q8s and (sh_gu is None or sh_dn is None or not shape.shared):
            raise ValueError("a q8s shared expert needs shared=True and both matrices")
        self.s = shape
        self.W, self.gu_w, self.dn_w = W, gu_w, dn_w
        self.sh_gu, self.sh_dn = sh_gu, sh_dn
        self.gu_stride = 2 * shape.ff * row_bytes(shape.wtype, shape.H)
        self.dn_stride = shape.H * row_bytes(shape.dn_type, shape.ff)

    @staticmethod
    def planar_from_gguf(shape: LayerShape, W: torch.Tensor, gu_gguf: torch.Tensor, dn_gguf: torch.Tensor,
                         sh_gu_gguf: torch.Tensor | None = None, sh_dn_gguf: torch.Tensor | None = None) -> "MoeLayer":
        """the GGUF blocks of n_routed experts (and, with sh_q8s, the shared expert's Q8_0 blocks) into the store"""
        s = shape
        gu = torch.empty_like(gu_gguf)
        dn = torch.empty_like(dn_gguf)
        store_pack(s.wtype, gu_gguf, gu, s.n_routed, 2 * s.ff, s.H)
        store_pack(s.dn_type, dn_gguf, dn, s.n_routed, s.H, s.ff)
        sh_gu = sh_dn = None
        if s.sh_q8s:
            sh_gu = Q8sMatrix.from_gguf(sh_gu_gguf, 2 * s.ff, s.H)
            sh_dn = Q8sMatrix.from_gguf(sh_dn_gguf, s.H, s.ff)
        return MoeLayer(s, W, gu, dn, sh_gu, sh_dn)

    @staticmethod
    def synthetic(shape: LayerShape, seed: int, device="cuda", chunk_experts: int = 64) -> "MoeLayer":
        """Seeded layer: router N(0, 0.02) fp32; experts N(0, 0.02) quantized by the library's quantizer and packed.
        A q8s shared expert takes expert E's values of the same streams, quantized to Q8_0."""
        s = shape
        E1 = s.n_routed
        W = torch.empty((s.E + 1, s.H), dtype=torch.float32, device=device)   # row E: the shared gate
        synth_normal(W, seed * 1000 + 1, 0.02)
        gu_stride = 2 * s.ff * row_bytes(s.wtype, s.H)
        dn_stride = s.H * row_bytes(s.dn_type, s.ff)
        gu = torch.empty(E1 * gu_stride, dtype=torch.uint8, device=device)
        dn = torch.empty(E1 * dn_stride, dtype=torch.uint8, device=device)
        vals = 2 * s.ff * s.H   # values per expert matrix (gate|up and down hold the same count)
        tmp = torch.empty(chunk_experts * vals, dtype=torch.float32, device=device)
        blk = torch.empty(chunk_experts * max(gu_stride, dn_stride), dtype=torch.uint8, device=device)
        for mat, (rows, cols, stride, dst, sd, wt) in enumerate(
                [(2 * s.ff, s.H, gu_stride, gu, seed * 1000 + 2, s.wtype), (s.H, s.ff, dn_stride, dn, seed * 1000 + 3, s.dn_type)]):
            for e0 in range(0, E1, chunk_experts):
                ne = min(chunk_experts, E1 - e0)
                t = tmp[: ne * rows * cols]
                synth_normal(t, sd, 0.02, offset=e0 * rows * cols)
                b = blk[: ne * stride]
                quantize_weights(wt, t.view(ne * rows, cols), b)
                store_pack(wt, b, dst[e0 * stride:(e0 + ne) * stride], ne, rows, cols)
        sh = [None, None]
        if s.sh_q8s:
            for mat, (rows, cols, sd) in enumerate([(2 * s.ff, s.H, seed * 1000 + 2), (s.H, s.ff, seed * 1000 + 3)]):
                t = tmp[: rows * cols]
                synth_normal(t, sd, 0.02, offset=s.E * rows * cols)
                b = blk[: rows * row_bytes(Q8_0, cols)]
                quantize_weights(Q8_0, t.view(rows, cols), b)
                sh[mat] = Q8sMatrix.from_gguf(b, rows, cols)
        del tmp, blk
        return MoeLayer(s, W, gu, dn, sh[0], sh[1])


class DecodeBuffers:
    """The decode window's buffers (src/engine.cu:174-206), T rows at most."""

    def __init__(self, shape: LayerShape, T: int, device="cuda"):
        s = shape
        P = T * s.K
        NP = P + (T if s.shared else 0)
        nj = P + 1
        i32 = dict(dtype=torch.int32, device=device)
        self.T = T
        self.xq = torch.empty(T * (s.H // 32) * 36, dtype=torch.uint8, device=device)
        self.logits = torch.empty((T, s.E + 1), dtype=torch.float32, device=device)
        self.topi = torch.empty((T, s.K), **i32)
        self.topw = torch.empty((T, s.K), dtype=torch.float32, device=device)
        self.jobs_gu = torch.zeros(nj * JOB_INTS, **i32)
        self.jobs_dn = torch.zeros(nj * JOB_INTS, **i32)
        self.njobs = torch.zeros(2, **i32)
        self.njobs_max = nj
        self.gu = torch.zeros((NP, 2 * s.ff), dtype=torch.float32, device=device)
        self.part = torch.zeros((NP, s.H), dtype=torch.float32, device=device)
        self.sh_hq = torch.zeros(T * (s.ff // 32) * 36, dtype=torch.uint8, device=device)   # the shared expert's h (q8_1)


def shared_q8s(L: "MoeLayer", T: int, xq, gu, hq, part) -> None:
    """the shared expert of a q8s layer for T rows, as src/engine.cu:942-944: q8s gate|up into gu rows P + t, SwiGLU to
    q8_1, q8s down into part rows P + t"""
    s = L.s
    P = T * s.K
    q8s_gemv(L.sh_gu, 2 * s.ff, s.H, xq, gu[P:P + T], 2 * s.ff, T)
    swiglu_stacked_q8_1(gu[P:P + T], hq, s.ff, T)
    q8s_gemv(L.sh_dn, s.H, s.ff, hq, part[P:P + T], s.H, T)


def decode_layer(L: MoeLayer, x: torch.Tensor, y: torch.Tensor, b: DecodeBuffers) -> None:
    """One decode window (T <= 16 rows) through the layer: the engine's ffn_half (src/engine.cu:933-978) on one GPU."""
    s = L.s
    T = x.shape[0]
    quantize_q8_1(x, b.xq)
    # a q8s shared expert is no job of the routed experts (src/engine.cu:936-945)
    router_route(L.W, x, b.logits, b.topi, b.topw, b.jobs_gu, b.jobs_dn, b.njobs, s.E, s.K, s.shared and not s.sh_q8s)
    moe_gate_up(L.gu_w, L.gu_stride, s.wtype, s.H, 2 * s.ff, b.jobs_gu, b.njobs, b.njobs_max, T, b.xq, b.gu)
    moe_down(L.dn_w, L.dn_stride, s.dn_type, s.ff, s.H, b.jobs_dn, b.njobs, b.njobs_max, T, b.gu, b.part)
    if s.sh_q8s:
        shared_q8s(L, T, b.xq, b.gu, b.sh_hq, b.part)
    moe_combine(b.part, b.topw, b.topi, b.logits, y, s.E, s.K, s.shared)


DECODE_PIECES = ["logits", "xq", "topi", "topw", "jobs_gu", "jobs_dn", "njobs", "gu", "hq_q", "hq_d", "hq_s", "y"]


class FusedDecode:
    """The fused decode path (sfnx_moe_decode): a window of up to T rows through a stack of layers, three launches a
    layer; owns its workspace and the layer table."""

    def __init__(self, layers: list, T: int, device="cuda"):
        s = layers[0].s
        self.s, self.T, self.layers = s, T, layers
        off = (C.c_size_t * 13)()
        total = lib().sfnx_moe_decode_workspace(T, s.H, s.E, s.K, s.ff, off)
        self.off = list(off)
        self.ws = torch.zeros(total, dtype=torch.uint8, device=device)
        self.table = (_abi.LayerW * len(layers))(*[
            _abi.LayerW(L.W.data_ptr(), L.gu_w.data_ptr(), L.gu_stride, L.dn_w.data_ptr(), L.dn_stride) for L in layers])
        self.sh_table = None
        if s.sh_q8s:
            self.sh_table = (_abi.SharedQ8s * len(layers))(*[
                _abi.SharedQ8s(L.sh_gu.c, L.sh_dn.c) for L in layers])

    def __call__(self, x: torch.Tensor, norm: bool = True, eps: float = 1e-6, layer0: int = 0,
                 n_layers: int | None = None, phases: int = 0) -> None:
        s = self.s
        n = len(self.layers) - layer0 if n_layers is None else n_layers
        table = C.cast(self.table, C.c_void_p).value + layer0 * C.sizeof(_abi.LayerW)
        if self.sh_table is not None:
            sh = C.cast(self.sh_table, C.c_void_p).value + layer0 * C.sizeof(_abi.SharedQ8s)
            check(lib().sfnx_moe_decode_q8s(table, sh, n, s.wtype, s.dn_type, s.H, s.E, s.K, s.ff, _p(x), x.shape[0],
                                            int(norm), eps, _p(self.ws), self.ws.numel(), phases, _st()))
            return
        check(lib().sfnx_moe_decode2(table, n, s.wtype, s.dn_type, s.H, s.E, s.K, s.ff, int(s.shared), _p(x), x.shape[0],
                                     int(norm), eps, _p(self.ws), self.ws.numel(), phases, _st()))

    def piece(self, name: str, dtype, shape) -> torch.Tensor:
        """a view of one workspace piece (the last layer's value)"""
        i = DECODE_PIECES.index(name)
        n = 1
        for d in shape:
            n *= d
        nbytes = n * torch.tensor([], dtype=dtype).element_size()
        return self.ws[self.off[i]: self.off[i] + nbytes].view(dtype).view(*shape)


class PrefillBuffers:
    """The prompt path's buffers for C tokens (src/prefill.cu:1145-1180)."""

    def __init__(self, shape: LayerShape, C: int, device="cuda"):
        s = shape
        P = C * s.K
        NP = P + (C if s.shared else 0)
        self.C = C
        self.cap = P // 64 + s.E + (C + 63) // 64 + 1
        i32 = dict(dtype=torch.int32, device=device)
        self.xq = torch.empty(C * (s.H // 32) * 36, dtype=torch.uint8, device=device)
        self.logits = torch.empty((C, s.E + 1), dtype=torch.float32, device=device)
        self.topi = torch.empty((C, s.K), **i32)
        self.topw = torch.empty((C, s.K), dtype=torch.float32, device=device)
        self.cnt = torch.zeros(s.E, **i32)
        self.jbase = torch.zeros(s.E, **i32)
        self.jobs_gu = torch.zeros(self.cap * BIGJOB_INTS, **i32)
        self.jobs_dn = torch.zeros(self.cap * BIGJOB_INTS, **i32)
        self.njobs = torch.zeros(2, **i32)
        self.gu = torch.zeros((NP, 2 * s.ff), dtype=torch.float32, device=device)
        self.part = torch.zeros((NP, s.H), dtype=torch.float32, device=device)
        self.xh = torch.zeros((C, s.H), dtype=torch.float16, device=device)
        self.h16 = torch.zeros((NP, s.ff), dtype=torch.float16, device=device)
        if s.sh_q8s:   # staging for the dense shared matrices (the reference's p.wh, sized for their f16 values)
            self.wh = torch.empty(2 * s.ff * s.H, dtype=torch.float16, device=device)


def prefill_route(L: "MoeLayer", x: torch.Tensor, b: "PrefillBuffers", bias: torch.Tensor | None = None,
                  xh: bool = False) -> None:
    """the prompt path's routing: router logits (and, with xh, b.xh = f16(x) from the same read), an optional bias on
    the routed logits (the benchmark's skew), then top-k and the BigJob permutation (src/prefill.cu:1163-1167)"""
    s = L.s
    if xh:
        router_logits_xh(L.W, x, b.logits, b.xh)
    else:
        router_logits(L.W, x, b.logits)
    if bias is not None:
        b.logits[:, : s.E] += bias
    pf_route(b.logits, b.topi, b.topw, b.cnt, b.jbase, b.jobs_gu, b.jobs_dn, b.njobs, s.E, s.K, s.shared and not s.sh_q8s)


def pf_dense(W: "Q8sMatrix", rows: int, cols: int, xh, out, ldo: int, wh) -> None:
    """src/prefill.cu:407-417 pf_dense_xh: out rows (stride ldo) = f16(W) . xh rows, fp32, on the matrix-core kernels;
    wh (the reference's staging buffer) receives W repacked for them (rows * cols * 34 / 32 bytes at least)"""
    check(lib().sfnx_pf_dense(W.ptr(), rows, cols, _p(xh), xh.shape[0], _p(out), ldo, _p(wh), wh.numel() * wh.element_size(), _st()))


def prefill_shared(L: "MoeLayer", b: "PrefillBuffers") -> None:
    """a q8s layer's shared expert for the chunk as the reference runs it (src/prefill.cu:1173-1177): its gate|up as one
    f16 GEMM of the dequantized Q8_0 rows (pf_dense_xh), SwiGLU to f16, its down likewise into part rows P + t; needs
    b.xh"""
    s = L.s
    C = b.C
    P = C * s.K
    pf_dense(L.sh_gu, 2 * s.ff, s.H, b.xh, b.gu[P:P + C], 2 * s.ff, b.wh)
    check(lib().sfnx_swiglu_h16(_p(b.gu[P:P + C]), s.ff, C, _p(b.h16[P:P + C]), _st()))
    pf_dense(L.sh_dn, s.H, s.ff, b.h16[P:P + C], b.part[P:P + C], s.H, b.wh)


def prefill_experts_mma(L: "MoeLayer", x: torch.Tensor, y: torch.Tensor, b: "PrefillBuffers") -> None:
    """the routed experts on the matrix cores after prefill_route: f16 activations, gate|up, SwiGLU to f16, down, the
    combine (the reference's default prompt path, src/prefill.cu:1167-1171)"""
    s = L.s
    to_f16(x, b.xh)
    moe_gate_up_mma(L.gu_w, L.gu_stride, s.wtype, s.H, 2 * s.ff, b.jobs_gu, b.njobs, b.cap, b.xh, b.gu)
    swiglu_h16(b.gu, b.h16, s.ff)
    moe_down_mma(L.dn_w, L.dn_stride, s.dn_type, s.ff, s.H, b.jobs_dn, b.njobs, b.cap, b.h16, b.part)
    if s.sh_q8s:
        prefill_shared(L, b)
    moe_combine(b.part, b.topw, b.topi, b.logits, y, s.E, s.K, s.shared)


def prefill_layer_mma(L: "MoeLayer", x: torch.Tensor, y: torch.Tensor, b: "PrefillBuffers",
                      bias: torch.Tensor | None = None) -> None:
    """A prompt chunk (or a verify window of many rows) through the whole layer on the matrix cores: routing, f16
    activations, gate|up with SwiGLU fused into its epilogue, down, the combine (src/prefill.cu:1145-1180)"""
    s = L.s
    prefill_route(L, x, b, bias, xh=True)   # the f16 activations b.xh from the router's read of x
    moe_gate_up_swiglu_mma(L.gu_w, L.gu_stride, s.wtype, s.H, s.ff, b.jobs_gu, b.njobs, b.cap, b.xh, b.h16)
    moe_down_mma(L.dn_w, L.dn_stride, s.dn_type, s.ff, s.H, b.jobs_dn, b.njobs, b.cap, b.h16, b.part)
    if s.sh_q8s:
        prefill_shared(L, b)
    moe_combine(b.part, b.topw, b.topi, b.logits, y, s.E, s.K, s.shared)


def prefill_layer_q8(L: MoeLayer, x: torch.Tensor, y: torch.Tensor, b: PrefillBuffers) -> None:
    """A prompt chunk through the layer on the int8 (q8_1) arithmetic, FNX_PF_MOE_Q8 (src/prefill.cu:1156-1166)."""
    s = L.s
    quantize_q8_1(x, b.xq)
    router_logits(L.W, x, b.logits)
    pf_route(b.logits, b.topi, b.topw, b.cnt, b.jbase, b.jobs_gu, b.jobs_dn, b.njobs, s.E, s.K, s.shared and not s.sh_q8s)
    moe_gate_up_big(L.gu_w, L.gu_stride, s.wtype, s.H, 2 * s.ff, b.jobs_gu, b.njobs, b.cap, b.xq, b.gu)
    moe_down_big(L.dn_w, L.dn_stride, s.dn_type, s.ff, s.H, b.jobs_dn, b.njobs, b.cap, b.gu, b.part)
    if s.sh_q8s:   # the reference's shared expert is the f16 dense path on this path too (src/prefill.cu:1173-1177)
        to_f16(x, b.xh)
        prefill_shared(L, b)
    moe_combine(b.part, b.topw, b.topi, b.logits, y, s.E, s.K, s.shared)


# ---------------------------------------------------------------------------------------------------- hc read
HC_PIECES = ["part", "ssp", "loq", "lod", "rs"]


class HcRead:
    """The hyper-connection read that produces the MoE half's input (src/kernels.cu:1054 hc_read, src/hc.cuh): one read's
    weights on the device (w_norm [HC N] f32; the down and up Q8S matrices as int8 values and f16 scale bits; the bf16
    inject rows or None) and a workspace for windows of up to 16 rows."""

    def __init__(self, N: int, HC: int, LR: int, w_norm, down_q, down_d, up_q, up_d, w_inj=None, device="cuda"):
        self.N, self.HC, self.LR = N, HC, LR
        dev = lambda a, dt: torch.as_tensor(a).to(device=device, dtype=dt).contiguous()
        self.w_norm = dev(w_norm, torch.float32)
        self.dq, self.uq = dev(down_q, torch.int8), dev(up_q, torch.int8)
        self.dd = dev(torch.as_tensor(down_d).view(torch.int16), torch.int16)
        self.ud = dev(torch.as_tensor(up_d).view(torch.int16), torch.int16)
        self.w_inj = None if w_inj is None else dev(torch.as_tensor(w_inj).view(torch.int16), torch.int16)
        off = (C.c_size_t * 6)()
        total = lib().sfnx_hc_workspace(N, HC, LR, off)
        self.off = list(off)
        self.ws = torch.zeros(total, dtype=torch.uint8, device=device)

    def __call__(self, R, mixed, xq=None, bo=None, inj_prev=None, inject=None, eps: float = 1e-6) -> None:
        """R [T][HC N] (R' written back when bo is given), mixed [T][N] out, xq [T][N/32] q8_1 out (or None)"""
        T = R.shape[0]
        check(lib().sfnx_hc_read(_p(R), _p(bo), _p(inj_prev), _p(self.w_norm), _p(self.dq), _p(self.dd), _p(self.uq),
                                 _p(self.ud), _p(self.w_inj), eps, _p(mixed), _p(inject), _p(xq), T, self.N, self.HC,
                                 self.LR, _p(self.ws), self.ws.numel(), _st()))

    def piece(self, name: str, dtype, shape) -> torch.Tensor:
        i = HC_PIECES.index(name)
        n = 1
        for d in shape:
            n *= d
        nbytes = n * torch.tensor([], dtype=dtype).element_size()
        return self.ws[self.off[i]: self.off[i] + nbytes].view(dtype).view(*shape)


# ---------------------------------------------------------------------------------------------------- GGUF files
class Gguf:
    """A GGUF model mapped read-only (src/gguf.hpp:46-88 Gguf): tensors by name, metadata by key."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().sfnx_gguf_open(str(path).encode(), C.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h:
            lib().sfnx_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, name: str):
        """(type, shape ne[0..n_dims), bytes as a numpy view of the mapping) or None when missing"""
        import numpy as np
        t = _abi.GgufTensor()
        r = lib().sfnx_gguf_find(self._h, name.encode(), C.byref(t))
        if r < 0:
            check(r)
        if r == 0:
            return None
        buf = (C.c_uint8 * t.nbytes).from_address(t.data) if t.nbytes else b""
        return t.type, tuple(t.ne[:t.n_dims]), np.frombuffer(buf, dtype=np.uint8)

    def names(self) -> list[str]:
        out = []
        for i in range(lib().sfnx_gguf_n_tensors(self._h)):
            n = C.c_char_p()
            check(lib().sfnx_gguf_tensor_at(self._h, i, C.byref(n), None))
            out.append(n.value.decode())
        return out

    def int(self, key: str):
        v = C.c_int64()
        r = lib().sfnx_gguf_int(self._h, key.encode(), C.byref(v))
        if r < 0:
            check(r)
        return v.value if r else None

    def float(self, key: str):
        v = C.c_double()
        r = lib().sfnx_gguf_float(self._h, key.encode(), C.byref(v))
        if r < 0:
            check(r)
        return v.value if r else None

    def str(self, key: str):
        v = C.c_char_p()
        r = lib().sfnx_gguf_str(self._h, key.encode(), C.byref(v))
        if r < 0:
            check(r)
        return v.value.decode() if r else None


def gguf_moe_layer(g: Gguf, layer: int, ff0: int = 0, ff1: int | None = None, K: int = 8, q8s: bool = False) -> "MoeLayer":
    """blk.<layer>'s experts, shared expert and router from a GGUF into a device MoeLayer (src/model.cpp:766-809).
    q8s: the shared expert as the reference loads it, dense Q8_0 matrices for the q8s sums (it must be Q8_0); else it
    joins the routed stores as expert E."""
    ti = g.tensor(f"blk.{layer}.ffn_gate_exps.weight")
    if ti is None:
        raise RuntimeError(f"gguf: blk.{layer}.ffn_gate_exps.weight is missing")
    wtype, (H, FF, E) = ti[0], ti[1]
    ff1 = FF if ff1 is None else ff1
    ffs = ff1 - ff0
    shared = all(g.tensor(f"blk.{layer}.{n}.weight") is not None
                 for n in ("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp", "ffn_gate_inp_shexp"))
    E1 = E + (1 if shared and not q8s else 0)
    gu_stride = 2 * ffs * row_bytes(wtype, H)
    td = g.tensor(f"blk.{layer}.ffn_down_exps.weight")
    dn_stride = H * row_bytes(td[0] if td is not None else wtype, ffs)
    gu = torch.empty(E1 * gu_stride, dtype=torch.uint8, device="cuda")
    dn = torch.empty(E1 * dn_stride, dtype=torch.uint8, device="cuda")
    W = torch.zeros((E + 1, H), dtype=torch.float32, device="cuda")   # row E: the shared gate (zero without one)
    info = (C.c_int * 6)()
    sh_gu = sh_dn = None
    if q8s:
        sh_gu, sh_dn = Q8sMatrix(2 * ffs, H), Q8sMatrix(H, ffs)
        check(lib().sfnx_gguf_moe_layer_q8s(g._h, layer, ff0, ff1, _p(gu), gu_stride, gu.numel(), _p(dn), dn_stride,
                                            dn.numel(), _p(W), W.shape[0], sh_gu.ptr(), sh_dn.ptr(), info, _st()))
    else:
        check(lib().sfnx_gguf_moe_layer(g._h, layer, ff0, ff1, _p(gu), gu_stride, gu.numel(), _p(dn), dn_stride, dn.numel(),
                                        _p(W), W.shape[0], info, _st()))
    s = LayerShape(H=H, E=E, K=K, ff=ffs, wtype=wtype, shared=shared, dn_wtype=None if info[5] == wtype else info[5],
                   sh_q8s=q8s)
    return MoeLayer(s, W, gu, dn, sh_gu, sh_dn)


__all__ = [n for n in dir() if not n.startswith("_")] + ["_abi"]


# ---------------------------------------------------------------------------------------------------- expert cache
class ExpertCache:
    """src/model.hpp:95-116 ExpertCache over a stack of layers of one expert size: every expert (the shared one among
    them when it is expert E of the stores) copied to page-locked host memory the GPU reads, n_slots VRAM slots in one
    pool, the tables ep_gu / ep_dn pointing at each expert's host copy until a plan gives it a slot.  The slots start
    empty (owner -1, ref 0), the hand at slot 0; the reference fills them at load with the hottest experts by a profile.
    layer_view(l) is layer l with its stores replaced by its rows of the tables (stride 0)."""

    def __init__(self, layers: list, n_slots: int, device="cuda"):
        import copy
        import numpy as np
        L0 = layers[0]
        self.layers, self.n_layers = layers, len(layers)
        self.n_experts = L0.gu_w.numel() // L0.gu_stride
        self.gu_bytes, self.dn_bytes = L0.gu_stride, L0.dn_stride
        for L in layers:
            if (L.gu_stride, L.dn_stride, L.gu_w.numel() // L.gu_stride) != (self.gu_bytes, self.dn_bytes, self.n_experts):
                raise ValueError("one pool: every layer's experts must have the same sizes")
        NL, E = self.n_layers, self.n_experts
        self.slot_bytes = self.gu_bytes + self.dn_bytes
        self.pool = torch.zeros(n_slots * self.slot_bytes, dtype=torch.uint8, device=device)
        self._host = []
        host_gu, host_dn = [], []
        for L in layers:
            for src, nbytes, dst in ((L.gu_w, self.gu_bytes, host_gu), (L.dn_w, self.dn_bytes, host_dn)):
                h, d = C.c_void_p(), C.c_void_p()
                check(lib().sfnx_host_alloc(E * nbytes, C.byref(h), C.byref(d)))
                self._host.append(h.value)
                arr = np.ctypeslib.as_array((C.c_uint8 * (E * nbytes)).from_address(h.value))
                arr[:] = src[: E * nbytes].cpu().numpy()
                dst += [d.value + e * nbytes for e in range(E)]
        i64 = dict(dtype=torch.int64, device=device)
        self.host_gu, self.host_dn = torch.tensor(host_gu, **i64), torch.tensor(host_dn, **i64)
        self.ep_gu, self.ep_dn = self.host_gu.clone(), self.host_dn.clone()
        self.slot_of = torch.full((NL * E,), -1, dtype=torch.int32, device=device)
        self.owner = torch.full((n_slots,), -1, dtype=torch.int32, device=device)
        self.ref = torch.zeros(n_slots, dtype=torch.uint8, device=device)
        self.hand = torch.zeros(_abi.EC_POOLS, dtype=torch.int32, device=device)
        self.status = torch.zeros(2, dtype=torch.int32, device=device)
        c = _abi.ExpertCacheC()
        c.n_slots, c.n_pools, c.n_layers, c.n_experts = n_slots, 1, NL, E
        c.s0[0], c.n[0], c.slot_bytes[0], c.dn_off[0], c.pool[0] = 0, n_slots, self.slot_bytes, self.gu_bytes, _p(self.pool)
        c.ep_gu, c.ep_dn, c.host_gu, c.host_dn = _p(self.ep_gu), _p(self.ep_dn), _p(self.host_gu), _p(self.host_dn)
        c.slot_of, c.owner, c.ref, c.hand = _p(self.slot_of), _p(self.owner), _p(self.ref), _p(self.hand)
        c.status = _p(self.status)
        self.c = c
        torch.cuda.synchronize()
        self._views = []
        for l, L in enumerate(layers):
            v = copy.copy(L)
            v.gu_w, v.gu_stride = self.ep_gu[l * E:(l + 1) * E], 0
            v.dn_w, v.dn_stride = self.ep_dn[l * E:(l + 1) * E], 0
            self._views.append(v)

    def layer_view(self, l: int) -> "MoeLayer":
        return self._views[l]

    def host_misses(self) -> tuple[int, int]:
        """(the misses the last plan left on their host copies, their running total); synchronises"""
        v = self.status.cpu().tolist()
        return int(v[0]), int(v[1])

    def plan(self, jobs, njobs, layer: int, out_list) -> None:
        check(lib().sfnx_cache_plan(_p(jobs), _p(njobs), layer, C.byref(self.c), _p(out_list), _st()))

    def copy(self, out_list) -> None:
        check(lib().sfnx_cache_copy(C.byref(self.c), 0, _p(out_list), _st()))

    def moe_cache(self, layer: int, out_list, jobs=None, njobs=None) -> None:
        """src/kernels.cu:1659-1668 moe_cache: the plan (when jobs is given) and the copy-in"""
        check(lib().sfnx_moe_cache(layer, self.gu_bytes, self.dn_bytes, C.byref(self.c), _p(out_list), _p(jobs), _p(njobs),
                                   _st()))

    def close(self) -> None:
        torch.cuda.synchronize()
        for h in self._host:
            check(lib().sfnx_host_free(h))
        self._host = []

    def __del__(self):
        try:
            if self._host:
                self.close()
        except Exception:
            pass


def decode_layer_cached(cache: ExpertCache, l: int, x: torch.Tensor, y: torch.Tensor, b: DecodeBuffers, out_list,
                        plan_in_router: bool = True) -> None:
    """decode_layer with the layer's experts behind the expert cache (src/engine.cu:947-971): the routing with the
    window's slots planned in its last block (or, plan_in_router=False, the plan as a launch of its own), the planned
    experts copied in (moe_cache), then the expert calls through the layer's tables"""
    V = cache.layer_view(l)
    s = V.s
    T = x.shape[0]
    quantize_q8_1(x, b.xq)
    shared = s.shared and not s.sh_q8s
    if plan_in_router:
        router_route(V.W, x, b.logits, b.topi, b.topw, b.jobs_gu, b.jobs_dn, b.njobs, s.E, s.K, shared,
                     plan=(cache, l, out_list))
        cache.moe_cache(l, out_list)
    else:
        router_route(V.W, x, b.logits, b.topi, b.topw, b.jobs_gu, b.jobs_dn, b.njobs, s.E, s.K, shared)
        cache.moe_cache(l, out_list, b.jobs_gu, b.njobs)
    moe_gate_up(V.gu_w, 0, s.wtype, s.H, 2 * s.ff, b.jobs_gu, b.njobs, b.njobs_max, T, b.xq, b.gu)
    moe_down(V.dn_w, 0, s.dn_type, s.ff, s.H, b.jobs_dn, b.njobs, b.njobs_max, T, b.gu, b.part)
    if s.sh_q8s:
        shared_q8s(V, T, b.xq, b.gu, b.sh_hq, b.part)
    moe_combine(b.part, b.topw, b.topi, b.logits, y, s.E, s.K, s.shared)
