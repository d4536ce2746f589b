"""A small GGUF v3 writer for the tests (the public GGUF layout: header, key/value pairs, tensor infos, aligned data),
so that the library's reader and layer loader can be checked on files whose every byte the test chose."""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)


def _s(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
           F64: "<d"}
    if t == STR:
        return _s(v.encode())
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(fmt[t], v)


def write_gguf(path, kv: list, tensors: list, alignment: int = 32, version: int = 3, bad_magic: bool = False) -> None:
    """kv: [(key, type, value)]; tensors: [(name, ggml type, ne (ne[0] first), bytes)]"""
    head = (b"GGUX" if bad_magic else b"GGUF") + struct.pack("<IQQ", version, len(tensors), len(kv))
    for k, t, v in kv:
        head += _s(k.encode()) + struct.pack("<I", t) + _value(t, v)
    off = 0
    offs = []
    for name, gt, ne, data in tensors:
        offs.append(off)
        head += _s(name.encode()) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", gt, off)
        off += (len(data) + alignment - 1) // alignment * alignment
    pad = (-len(head)) % alignment
    body = b""
    for (name, gt, ne, data), o in zip(tensors, offs):
        body += bytes(data) + b"\0" * ((-len(data)) % alignment)
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad + body)


def moe_layer_tensors(layer: int, W: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray, wtype: int,
                      H: int, E: int, ff: int, shared=None, dn_type: int | None = None, sh_type: int | None = None) -> list:
    """the tensors of one MoE layer as a Qwen3-MoE style GGUF names them: per-expert GGUF blocks (gate, up: [E][ff]
    rows of H; down: [E][H] rows of ff), router f32 [E][H], and optionally (gate_s, up_s, down_s, gate_row), the shared
    matrices in sh_type when given (Q8_0 as the reference's models carry them), else in the routed types"""
    p = f"blk.{layer}."
    dt = wtype if dn_type is None else dn_type
    t = [(p + "ffn_gate_exps.weight", wtype, (H, ff, E), gate.tobytes()),
         (p + "ffn_up_exps.weight", wtype, (H, ff, E), up.tobytes()),
         (p + "ffn_down_exps.weight", dt, (ff, H, E), down.tobytes()),
         (p + "ffn_gate_inp.weight", 0, (H, E), np.ascontiguousarray(W[:E], np.float32).tobytes())]
    if shared is not None:
        gs, us, ds, grow = shared
        st, sdt = (wtype, dt) if sh_type is None else (sh_type, sh_type)
        t += [(p + "ffn_gate_shexp.weight", st, (H, ff), gs.tobytes()),
              (p + "ffn_up_shexp.weight", st, (H, ff), us.tobytes()),
              (p + "ffn_down_shexp.weight", sdt, (ff, H), ds.tobytes()),
              (p + "ffn_gate_inp_shexp.weight", 0, (H, 1), np.ascontiguousarray(grow, np.float32).tobytes())]
    return t
