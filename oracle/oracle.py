"""numpy bindings of the CPU oracle (liborc.so).  TEST INFRASTRUCTURE ONLY: imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker, never by the sfnx_amd package.

Each wrapper names the C function it calls; the C functions cite the reference lines they restate.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liborc.so"

Q4_0, Q5_1, Q8_0, Q4_K, Q5_K = 2, 7, 8, 12, 13
Q4K_BYTES, Q5K_BYTES, Q40_BYTES, Q51_BYTES, Q80_BYTES, Q81_BYTES = 144, 176, 18, 24, 34, 36
NAMES = {Q4_0: 'q4_0', Q5_1: 'q5_1', Q8_0: 'q8_0', Q4_K: 'q4_k', Q5_K: 'q5_k'}
MAXT, PF_JOB = 16, 64

JOB_DTYPE = np.dtype([("w", "<i4"), ("n", "<i4"), ("y", "<i4", MAXT), ("out", "<i4", MAXT)])
BIGJOB_DTYPE = np.dtype([("w", "<i4"), ("n", "<i4"), ("y", "<i4", PF_JOB), ("out", "<i4", PF_JOB)])


class Layer(C.Structure):
    _fields_ = [
        ("W", C.c_void_p), ("gu_w", C.c_void_p), ("gu_stride", C.c_size_t), ("dn_w", C.c_void_p),
        ("dn_stride", C.c_size_t), ("type", C.c_int), ("H", C.c_int), ("E", C.c_int), ("K", C.c_int),
        ("ff", C.c_int), ("shared", C.c_int), ("dn_type", C.c_int), ("sh_gu", C.c_void_p), ("sh_dn", C.c_void_p),
    ]


def build() -> Path:
    """make -C oracle (gcc + OpenMP)."""
    r = subprocess.run(["make", "-s", "-C", str(HERE)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stderr)
    return LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        vp, i32, i64, sz, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_float
        sig = {
            "orc_f16_to_f32": (f32, [C.c_uint16]),
            "orc_f32_to_f16": (C.c_uint16, [f32]),
            "orc_f16_fma": (C.c_uint16, [C.c_uint16] * 3),
            "orc_f16_mul": (C.c_uint16, [C.c_uint16] * 2),
            "orc_synth_normal": (None, [vp, sz, C.c_uint64, C.c_uint64, f32]),
            "orc_quantize_q4_k": (None, [vp, vp, i64, i32]),
            "orc_quantize_q8_0": (None, [vp, vp, i64, i32]),
            "orc_quantize_q5_k": (None, [vp, vp, i64, i32]),
            "orc_dequant_q5_k": (None, [vp, vp, i64, i32]),
            "orc_dequant_q5_k_f16": (None, [vp, vp, i64, i32]),
            "orc_dot_q5_k": (f32, [vp, vp, i32]),
            "orc_dot_q8s": (f32, [vp, vp, i32]),
            "orc_hc_read": (None, [vp, vp, vp, vp, vp, vp, vp, vp, vp, f32, i32, i32, i32, i32, vp, vp, vp, vp, vp]),
            "orc_quantize_q4_0": (None, [vp, vp, i64, i32]),
            "orc_dequant_q4_0": (None, [vp, vp, i64, i32]),
            "orc_dequant_q4_0_f16": (None, [vp, vp, i64, i32]),
            "orc_dot_q4_0": (f32, [vp, vp, i32]),
            "orc_quantize_q5_1": (None, [vp, vp, i64, i32]),
            "orc_dequant_q5_1": (None, [vp, vp, i64, i32]),
            "orc_dequant_q5_1_f16": (None, [vp, vp, i64, i32]),
            "orc_dot_q5_1": (f32, [vp, vp, i32]),
            "orc_q4k_scale_min": (None, [vp, i32, vp, vp]),
            "orc_dequant_q4_k": (None, [vp, vp, i64, i32]),
            "orc_dequant_q4_k_f16": (None, [vp, vp, i64, i32]),
            "orc_dequant_q8_0": (None, [vp, vp, i64, i32]),
            "orc_dequant_q8_0_f16": (None, [vp, vp, i64, i32]),
            "orc_quantize_q8_1": (None, [vp, vp, i32, i32]),
            "orc_router_logits": (None, [vp, vp, vp, i32, i32, i32]),
            "orc_router_logits_mm": (None, [vp, vp, vp, i32, i32, i32]),
            "orc_router_logits_prompt": (None, [vp, vp, vp, i32, i32, i32]),
            "orc_topk": (i32, [vp, i32, i32, i32, i32, vp, vp]),
            "orc_jobs_decode": (i32, [vp, i32, i32, i32, i32, vp, vp]),
            "orc_jobs_prefill": (i32, [vp, i32, i32, i32, i32, vp, vp, vp, vp]),
            "orc_dot_q4_k": (f32, [vp, vp, i32]),
            "orc_dot_q8_0": (f32, [vp, vp, i32]),
            "orc_swiglu_q8_1": (None, [vp, i32, vp]),
            "orc_layer_decode": (None, [C.POINTER(Layer), vp, i32, vp, vp, vp, vp, vp, vp, i32]),
            "orc_layer_prompt": (None, [C.POINTER(Layer), vp, i32, vp, vp, vp, vp, vp, vp, i32]),
            "orc_mma_matvec": (None, [vp, i32, i32, i32, vp, vp]),
            "orc_swiglu_h16": (None, [vp, i32, vp]),
            "orc_time_layer_decode": (C.c_double, [C.POINTER(Layer), vp, i32, i32, sz, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the oracle must be contiguous"
    return a.ctypes.data


def row_bytes(t: int, cols: int) -> int:
    return {Q4_K: cols // 256 * Q4K_BYTES, Q5_K: cols // 256 * Q5K_BYTES, Q4_0: cols // 32 * Q40_BYTES,
            Q5_1: cols // 32 * Q51_BYTES}.get(t, cols // 32 * Q80_BYTES)


def _by_type(t: int, q4k: str, q5k: str, q80: str):
    """the oracle function for type t (the names given are the K-quant / Q8_0 ones; Q4_0 / Q5_1 follow their pattern)"""
    if t in (Q4_0, Q5_1):
        return getattr(lib(), q80.replace("q8_0", NAMES[t]))
    return getattr(lib(), {Q4_K: q4k, Q5_K: q5k}.get(t, q80))


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().orc_f32_to_f16(f)


def synth(n: int, seed: int, std: float, offset: int = 0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_synth_normal(_p(out), n, seed, offset, std)
    return out


def quantize(t: int, x: np.ndarray) -> np.ndarray:
    rows, cols = x.shape
    out = np.empty(rows * row_bytes(t, cols), np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    _by_type(t, 'orc_quantize_q4_k', 'orc_quantize_q5_k', 'orc_quantize_q8_0')(_p(x), _p(out), rows, cols)
    return out


def dequant(t: int, blocks: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    _by_type(t, 'orc_dequant_q4_k', 'orc_dequant_q5_k', 'orc_dequant_q8_0')(_p(blocks), _p(out), rows, cols)
    return out


def dequant_f16(t: int, blocks: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), np.uint16)
    _by_type(t, 'orc_dequant_q4_k_f16', 'orc_dequant_q5_k_f16', 'orc_dequant_q8_0_f16')(_p(blocks), _p(out), rows, cols)
    return out


def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    rows, n = x.shape
    out = np.empty(rows * n // 32 * Q81_BYTES, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    lib().orc_quantize_q8_1(_p(x), _p(out), n, rows)
    return out


def router_logits(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    L, H = W.shape
    T = x.shape[0]
    out = np.empty((T, L), np.float32)
    lib().orc_router_logits(_p(W), _p(np.ascontiguousarray(x)), _p(out), T, H, L)
    return out


def router_logits_mm(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """the prompt path's router logits in the matrix-core kernel's summation order"""
    L, H = W.shape
    T = x.shape[0]
    out = np.empty((T, L), np.float32)
    lib().orc_router_logits_mm(_p(W), _p(np.ascontiguousarray(x)), _p(out), T, H, L)
    return out


ROUTER_MM_MIN_T = 512   # oracle.h ORC_ROUTER_MM_MIN_T


def router_logits_prompt(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """sfnx_router_logits' order for this many tokens: the matrix-core order from ROUTER_MM_MIN_T tokens, else the
    VALU kernel's (router_logits)"""
    L, H = W.shape
    T = x.shape[0]
    out = np.empty((T, L), np.float32)
    lib().orc_router_logits_prompt(_p(W), _p(np.ascontiguousarray(x)), _p(out), T, H, L)
    return out


def topk(logits: np.ndarray, E: int, K: int):
    T, ld = logits.shape
    topi = np.empty((T, K), np.int32)
    topw = np.empty((T, K), np.float32)
    missing = lib().orc_topk(_p(np.ascontiguousarray(logits, np.float32)), T, E, ld, K, _p(topi), _p(topw))
    return topi, topw, missing


def jobs_decode(topi: np.ndarray, K: int, E: int, shared: bool):
    T = topi.shape[0]
    gu = np.zeros(T * K + 1, JOB_DTYPE)
    dn = np.zeros(T * K + 1, JOB_DTYPE)
    n = lib().orc_jobs_decode(_p(np.ascontiguousarray(topi, np.int32)), T, K, E, int(shared), _p(gu), _p(dn))
    return gu[:n], dn[:n]


def jobs_prefill(topi: np.ndarray, K: int, E: int, shared: bool):
    C_ = topi.shape[0]
    cap = C_ * K // PF_JOB + E + (C_ + PF_JOB - 1) // PF_JOB + 1
    gu = np.zeros(cap, BIGJOB_DTYPE)
    dn = np.zeros(cap, BIGJOB_DTYPE)
    cnt = np.empty(E, np.int32)
    jbase = np.empty(E, np.int32)
    n = lib().orc_jobs_prefill(_p(np.ascontiguousarray(topi, np.int32)), C_, K, E, int(shared), _p(cnt), _p(jbase),
                               _p(gu), _p(dn))
    return cnt, jbase, gu[:n], dn[:n]


def dot(t: int, wrow: np.ndarray, yq: np.ndarray, K: int) -> float:
    f = _by_type(t, 'orc_dot_q4_k', 'orc_dot_q5_k', 'orc_dot_q8_0')
    return f(_p(np.ascontiguousarray(wrow)), _p(np.ascontiguousarray(yq)), K)


def dot_q8s(wrow: np.ndarray, yq: np.ndarray, K: int) -> float:
    """the shared expert's dense Q8_0 row dot, src/dense.cuh:24-154 (orc_dot_q8s)"""
    return lib().orc_dot_q8s(_p(np.ascontiguousarray(wrow)), _p(np.ascontiguousarray(yq)), K)


class HcWeights:
    """one hyper-connection read's weights (src/hc.cuh HcArgs): w_norm [HC N] f32, down Q8S (dq int8 [LR][HC N],
    dd f16 bits [LR][HC N / 32]), up Q8S (uq [HC N][LR], ud [HC N][LR / 32]), w_inj bf16 bits [HC][HC N] or None"""

    def __init__(self, N, HC, LR, w_norm, dq, dd, uq, ud, w_inj=None):
        self.N, self.HC, self.LR = N, HC, LR
        self.w_norm = np.ascontiguousarray(w_norm, np.float32)
        self.dq, self.dd = np.ascontiguousarray(dq, np.int8), np.ascontiguousarray(dd, np.uint16)
        self.uq, self.ud = np.ascontiguousarray(uq, np.int8), np.ascontiguousarray(ud, np.uint16)
        self.w_inj = None if w_inj is None else np.ascontiguousarray(w_inj, np.uint16)


def hc_read(w: HcWeights, R: np.ndarray, bo=None, inj_prev=None, eps: float = 1e-6):
    """src/hc.cuh:13-380 for T rows: returns mixed, inject, xq (q8_1), R' (R with bo folded in), part, ssp"""
    T = R.shape[0]
    D, NS, ROWS = w.HC * w.N, w.HC * w.N // 512, w.LR + w.HC
    R = np.array(R, np.float32, copy=True)
    mixed = np.empty((T, w.N), np.float32)
    inject = np.zeros((T, w.HC), np.float32)
    xq = np.empty(T * (w.N // 32) * Q81_BYTES, np.uint8)
    part = np.empty((T, NS, ROWS), np.float32)
    ssp = np.empty((T, NS), np.float32)
    bo_ = None if bo is None else np.ascontiguousarray(bo, np.float32)
    ij = None if inj_prev is None else np.ascontiguousarray(inj_prev, np.float32)
    lib().orc_hc_read(_p(R), _p(bo_), _p(ij), _p(w.w_norm), _p(w.dq), _p(w.dd), _p(w.uq), _p(w.ud), _p(w.w_inj), eps, T,
                      w.N, w.HC, w.LR, _p(mixed), _p(inject), _p(xq), _p(part), _p(ssp))
    return mixed, inject, xq, R, part, ssp


def swiglu_q8_1(gu_row: np.ndarray, ff: int) -> np.ndarray:
    out = np.empty(ff // 32 * Q81_BYTES, np.uint8)
    lib().orc_swiglu_q8_1(_p(np.ascontiguousarray(gu_row, np.float32)), ff, _p(out))
    return out


class LayerWeights:
    """A layer in GGUF block layout: router W [E+1][H] fp32, gate|up experts [E+1][2ff][H], down [E+1][H][ff]."""

    def __init__(self, W, gu_w, dn_w, wtype, H, E, K, ff, shared=True, dn_type=None, sh_gu=None, sh_dn=None):
        self.W = np.ascontiguousarray(W, np.float32)
        self.gu_w = np.ascontiguousarray(gu_w, np.uint8)
        self.dn_w = np.ascontiguousarray(dn_w, np.uint8)
        self.type, self.H, self.E, self.K, self.ff, self.shared = wtype, H, E, K, ff, shared
        self.dn_type = wtype if dn_type is None else dn_type
        self.gu_stride = 2 * ff * row_bytes(wtype, H)
        self.dn_stride = H * row_bytes(self.dn_type, ff)
        # a separate Q8_0 shared expert (GGUF blocks), computed with the reference's dense q8s arithmetic
        self.sh_gu = None if sh_gu is None else np.ascontiguousarray(sh_gu, np.uint8)
        self.sh_dn = None if sh_dn is None else np.ascontiguousarray(sh_dn, np.uint8)
        self.c = Layer(_p(self.W), _p(self.gu_w), self.gu_stride, _p(self.dn_w), self.dn_stride, wtype, H, E, K, ff,
                       int(shared), self.dn_type, _p(self.sh_gu), _p(self.sh_dn))


def layer_decode(L: LayerWeights, x: np.ndarray, nthreads: int = 0, prompt: bool = False):
    """Returns y, logits, topi, topw, gu, part (src/engine.cu:933-978's MoE half for T tokens); prompt: routed with the
    prompt path's router order (router_logits_prompt)."""
    T = x.shape[0]
    NP = T * L.K + (T if L.shared else 0)
    y = np.empty((T, L.H), np.float32)
    logits = np.empty((T, L.E + 1), np.float32)
    topi = np.empty((T, L.K), np.int32)
    topw = np.empty((T, L.K), np.float32)
    gu = np.zeros((NP, 2 * L.ff), np.float32)
    part = np.zeros((NP, L.H), np.float32)
    x = np.ascontiguousarray(x, np.float32)
    fn = lib().orc_layer_prompt if prompt else lib().orc_layer_decode
    fn(C.byref(L.c), _p(x), T, _p(y), _p(logits), _p(topi), _p(topw), _p(gu), _p(part), nthreads)
    return y, logits, topi, topw, gu, part


def mma_matvec(t: int, w: np.ndarray, n_in: int, n_out: int, x16: np.ndarray) -> np.ndarray:
    out = np.empty(n_out, np.float64)
    lib().orc_mma_matvec(_p(np.ascontiguousarray(w)), t, n_in, n_out, _p(np.ascontiguousarray(x16, np.uint16)), _p(out))
    return out


def swiglu_h16(gu_row: np.ndarray, ff: int) -> np.ndarray:
    out = np.empty(ff, np.uint16)
    lib().orc_swiglu_h16(_p(np.ascontiguousarray(gu_row, np.float32)), ff, _p(out))
    return out


def time_layer_decode(L: LayerWeights, x: np.ndarray, nthreads: int, reps: int, sweep_bytes: int):
    y = np.empty((1, L.H), np.float32)
    us = lib().orc_time_layer_decode(C.byref(L.c), _p(np.ascontiguousarray(x, np.float32)), nthreads, reps,
                                     sweep_bytes, _p(y))
    return us, y
