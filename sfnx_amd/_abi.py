"""ctypes bindings of the C ABI in include/sfnx_moe.h (libsfnx_moe.so, built in-tree by sfnx_amd/build.py).

Loading fails loudly when the library is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("SFNX_LIB", PKG / "libsfnx_moe.so"))   # SFNX_LIB: a library built elsewhere
HEADER = PKG.parent / "include" / "sfnx_moe.h"

Q4_0, Q5_1, Q8_0, Q4_K, Q5_K = 2, 7, 8, 12, 13
MAXT, PF_JOB = 16, 64
JOB_INTS = 2 + 2 * MAXT        # sfnx_job: w, n, y[16], out[16]
BIGJOB_INTS = 2 + 2 * PF_JOB   # sfnx_bigjob

vp, i32, i64, sz, f32, u32, u64 = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_float, C.c_uint32, C.c_uint64

SIGNATURES = {
    "sfnx_last_error": (C.c_char_p, []),
    "sfnx_abi_version": (i32, []),
    "sfnx_row_bytes": (sz, [u32, i32]),
    "sfnx_synth_normal": (i32, [vp, sz, u64, u64, f32, vp]),
    "sfnx_quantize_weights": (i32, [u32, vp, vp, i64, i32, vp]),
    "sfnx_store_pack": (i32, [u32, vp, vp, i64, i32, i32, vp]),
    "sfnx_store_unpack": (i32, [u32, vp, vp, i64, i32, i32, vp]),
    "sfnx_dequantize": (i32, [u32, vp, vp, i64, i32, i32, vp]),
    "sfnx_dequantize_f16": (i32, [u32, vp, vp, i64, i32, i32, vp]),
    "sfnx_quantize_q8_1": (i32, [vp, vp, i32, i32, vp]),
    "sfnx_router_route": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, i32, vp]),
    "sfnx_router_logits": (i32, [vp, vp, vp, i32, i32, i32, vp]),
    "sfnx_router_logits_xh": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "sfnx_pf_route": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, i32, vp]),
    "sfnx_moe_gate_up": (i32, [vp, sz, u32, i32, i32, vp, vp, i32, i32, vp, vp, vp]),
    "sfnx_moe_down": (i32, [vp, sz, u32, i32, i32, vp, vp, i32, i32, vp, vp, vp]),
    "sfnx_moe_gate_up_big": (i32, [vp, sz, u32, i32, i32, vp, vp, i32, vp, vp, vp]),
    "sfnx_moe_down_big": (i32, [vp, sz, u32, i32, i32, vp, vp, i32, vp, vp, vp]),
    "sfnx_moe_combine": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "sfnx_residual_rmsnorm": (i32, [vp, vp, vp, i32, i32, f32, vp]),
    "sfnx_kernel_clock": (i32, [i32]),
    "sfnx_kernel_clock_read": (i32, [vp]),
    "sfnx_moe_gate_up_mma": (i32, [vp, sz, u32, i32, i32, vp, vp, i32, vp, vp, vp]),
    "sfnx_swiglu_h16": (i32, [vp, i32, i32, vp, vp]),
    "sfnx_moe_gate_up_swiglu_mma": (i32, [vp, sz, u32, i32, i32, vp, vp, i32, vp, vp, vp]),
    "sfnx_moe_down_mma": (i32, [vp, sz, u32, i32, i32, vp, vp, i32, vp, vp, vp]),
    "sfnx_to_f16": (i32, [vp, vp, sz, vp]),
    "sfnx_moe_decode_workspace": (sz, [i32, i32, i32, i32, i32, vp]),
    "sfnx_moe_decode": (i32, [vp, i32, u32, i32, i32, i32, i32, i32, vp, i32, i32, f32, vp, sz, i32, vp]),
    "sfnx_moe_decode_noalloc": (i32, [vp, i32, u32, u32, i32, i32, i32, i32, i32, vp, i32, i32, f32, vp]),
    "sfnx_moe_decode2": (i32, [vp, i32, u32, u32, i32, i32, i32, i32, i32, vp, i32, i32, f32, vp, sz, i32, vp]),
    "sfnx_moe_decode_q8s": (i32, [vp, vp, i32, u32, u32, i32, i32, i32, i32, vp, i32, i32, f32, vp, sz, i32, vp]),
    "sfnx_q8s_gemv": (i32, [vp, i32, i32, vp, vp, i32, i32, vp]),
    "sfnx_q8s_split": (i32, [vp, i32, i32, vp, vp]),
    "sfnx_hc_workspace": (sz, [i32, i32, i32, vp]),
    "sfnx_pf_dense": (i32, [vp, i32, i32, vp, i32, vp, i32, vp, sz, vp]),
    "sfnx_hc_read": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, f32, vp, vp, vp, i32, i32, i32, i32, vp, sz, vp]),
    "sfnx_swiglu_stacked_q8_1": (i32, [vp, vp, i32, i32, vp]),
    "sfnx_q8s_swiglu_gemv": (i32, [vp, i32, i32, vp, vp, i32, i32, vp]),
    "sfnx_gguf_type_info": (i32, [u32, vp, vp]),
    "sfnx_gguf_open": (i32, [C.c_char_p, vp]),
    "sfnx_gguf_close": (None, [vp]),
    "sfnx_gguf_n_tensors": (i32, [vp]),
    "sfnx_gguf_tensor_at": (i32, [vp, i32, vp, vp]),
    "sfnx_gguf_find": (i32, [vp, C.c_char_p, vp]),
    "sfnx_gguf_int": (i32, [vp, C.c_char_p, vp]),
    "sfnx_gguf_float": (i32, [vp, C.c_char_p, vp]),
    "sfnx_gguf_str": (i32, [vp, C.c_char_p, vp]),
    "sfnx_gguf_moe_layer": (i32, [vp, i32, i32, i32, vp, sz, sz, vp, sz, sz, vp, i32, vp, vp]),
    "sfnx_gguf_moe_layer_q8s": (i32, [vp, i32, i32, i32, vp, sz, sz, vp, sz, sz, vp, i32, vp, vp, vp, vp]),
    "sfnx_host_alloc": (i32, [sz, vp, vp]),
    "sfnx_host_free": (i32, [vp]),
    "sfnx_cache_plan": (i32, [vp, vp, i32, vp, vp, vp]),
    "sfnx_router_route_plan": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, i32, vp, i32, vp, vp]),
    "sfnx_cache_copy": (i32, [vp, i32, vp, vp]),
    "sfnx_moe_cache": (i32, [i32, sz, sz, vp, vp, vp, vp, vp]),
}


class GgufTensor(C.Structure):
    """sfnx_gguf_tensor"""
    _fields_ = [("type", u32), ("n_dims", i32), ("ne", i64 * 4), ("data", vp), ("nbytes", sz), ("shard", i32)]


class LayerW(C.Structure):
    """sfnx_moe_layer_w"""
    _fields_ = [("W", vp), ("gu", vp), ("gu_stride", sz), ("dn", vp), ("dn_stride", sz)]


class Q8S(C.Structure):
    """sfnx_q8s (src/model.hpp:71-74 Q8S): int8 values q [rows][cols], f16 scale bits d [rows][cols / 32]"""
    _fields_ = [("q", vp), ("d", vp)]


class SharedQ8s(C.Structure):
    """sfnx_moe_shared_q8s"""
    _fields_ = [("gu", Q8S), ("dn", Q8S)]


EC_POOLS, EC_LAYERS = 4, 128


class ExpertCacheC(C.Structure):
    """sfnx_expert_cache"""
    _fields_ = [("n_slots", i32), ("n_pools", i32), ("n_layers", i32), ("n_experts", i32),
                ("pool_of", i32 * EC_LAYERS), ("s0", i32 * EC_POOLS), ("n", i32 * EC_POOLS),
                ("slot_bytes", sz * EC_POOLS), ("dn_off", sz * EC_POOLS), ("pool", vp * EC_POOLS),
                ("ep_gu", vp), ("ep_dn", vp), ("host_gu", vp), ("host_dn", vp),
                ("slot_of", vp), ("owner", vp), ("ref", vp), ("hand", vp), ("status", vp)]


def declared_symbols() -> list[str]:
    """Every function the C header declares."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(sfnx_[a-z0-9_]+)\s*\(", text)))


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() (or python sfnx_amd/build.py)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != 0:
        raise RuntimeError(lib().sfnx_last_error().decode())
