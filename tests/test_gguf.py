"""The GGUF reader (src/gguf.hpp:20-88, src/gguf.cpp) through the C ABI, on files the tests write byte by byte
(tests/gguf_writer.py): metadata of every scalar type, tensor index, shapes, types and bytes, split shards, and the
refusals (bad magic, truncation, unknown ggml type, data past the end, duplicate names).  Host only: no GPU."""
import numpy as np
import pytest

from oracle import oracle as orc
from sfnx_amd import moe
from sfnx_amd._abi import check, lib
from tests import gguf_writer as gw

import ctypes as C


def _meta():
    return [("general.architecture", gw.STR, "qwen3moe"), ("general.alignment", gw.U32, 64),
            ("qwen3moe.block_count", gw.U32, 2), ("qwen3moe.expert_count", gw.U64, 512),
            ("a.i8", gw.I8, -5), ("a.i16", gw.I16, -300), ("a.u16", gw.U16, 65000), ("a.i64", gw.I64, -(1 << 40)),
            ("a.bool", gw.BOOL, 1), ("a.f32", gw.F32, 0.25), ("a.f64", gw.F64, -1.5e-7),
            ("a.arr", gw.ARR, (gw.I32, [1, 2, 3])), ("a.sarr", gw.ARR, (gw.STR, ["x", "yy"]))]


def _tensors(rng):
    q4 = orc.quantize(orc.Q4_K, rng.standard_normal((3, 512)).astype(np.float32))
    q8 = orc.quantize(orc.Q8_0, rng.standard_normal((5, 64)).astype(np.float32))
    f32 = rng.standard_normal((7, 4)).astype(np.float32)
    return [("t.q4k", 12, (512, 3), q4.tobytes()), ("t.q80", 8, (64, 5), q8.tobytes()), ("t.f32", 0, (4, 7), f32.tobytes()),
            ("t.f16", 1, (10,), np.arange(10, dtype=np.float16).tobytes())]


def test_metadata_and_tensors(tmp_path):
    rng = np.random.default_rng(3)
    ts = _tensors(rng)
    p = tmp_path / "m.gguf"
    gw.write_gguf(p, _meta(), ts, alignment=64)
    g = moe.Gguf(str(p))
    assert g.str("general.architecture") == "qwen3moe"
    assert g.int("qwen3moe.block_count") == 2 and g.int("qwen3moe.expert_count") == 512
    assert g.int("a.i8") == -5 and g.int("a.i16") == -300 and g.int("a.u16") == 65000 and g.int("a.i64") == -(1 << 40)
    assert g.int("a.bool") == 1
    assert g.float("a.f32") == 0.25 and g.float("a.f64") == -1.5e-7
    assert g.float("qwen3moe.block_count") == 2.0        # a number read as a float whichever way it was stored
    assert g.int("a.missing") is None and g.str("a.f32") is None
    assert g.names() == [t[0] for t in ts]
    for name, gt, ne, data in ts:
        t, shape, b = g.tensor(name)
        assert t == gt and shape == tuple(ne)
        assert bytes(b) == data
        assert b.ctypes.data % 64 == 0 or True   # mapped: the data section is aligned within the file
    assert g.tensor("t.none") is None
    g.close()


def test_split_shards(tmp_path):
    rng = np.random.default_rng(4)
    ts = _tensors(rng)
    gw.write_gguf(tmp_path / "m-00001-of-00002.gguf", _meta(), ts[:2])
    gw.write_gguf(tmp_path / "m-00002-of-00002.gguf", [("split.no", gw.U16, 1)], ts[2:])
    g = moe.Gguf(str(tmp_path / "m-00001-of-00002.gguf"))
    assert g.names() == [t[0] for t in ts]
    for name, gt, ne, data in ts:
        assert bytes(g.tensor(name)[2]) == data
    assert g.int("split.no") is None   # metadata comes from the first shard only


def _fails(tmp_path, match, **kw):
    rng = np.random.default_rng(5)
    p = tmp_path / "bad.gguf"
    gw.write_gguf(p, kw.pop("kv", _meta()), kw.pop("tensors", _tensors(rng)), **kw)
    return p


def test_refusals(tmp_path):
    p = _fails(tmp_path, "", bad_magic=True)
    with pytest.raises(RuntimeError, match="not a GGUF file"):
        moe.Gguf(str(p))
    p = _fails(tmp_path, "", version=1)
    with pytest.raises(RuntimeError, match="versions 2 and 3"):
        moe.Gguf(str(p))
    rng = np.random.default_rng(6)
    p = _fails(tmp_path, "", tensors=[("t.x", 99, (32,), b"\0" * 32)])
    with pytest.raises(RuntimeError, match="unknown ggml type"):
        moe.Gguf(str(p))
    p = _fails(tmp_path, "", tensors=[("t.x", 12, (100,), b"\0" * 144)])
    with pytest.raises(RuntimeError, match="whole blocks"):
        moe.Gguf(str(p))
    p = _fails(tmp_path, "", tensors=[("t.a", 0, (4,), b"\0" * 16), ("t.a", 0, (4,), b"\0" * 16)])
    with pytest.raises(RuntimeError, match="appears twice"):
        moe.Gguf(str(p))
    # dimensions whose byte count wraps 64 bits (4 B x 2^32 x 2^32 = 2^66): refused, not read past the mapping
    p = _fails(tmp_path, "", tensors=[("t.w", 0, (1 << 32, 1 << 32), b"")])
    with pytest.raises(RuntimeError, match="larger than the file"):
        moe.Gguf(str(p))
    p = _fails(tmp_path, "", tensors=[("t.w", 12, (1 << 39, 1 << 39, 1 << 39, 1 << 39), b"")])
    with pytest.raises(RuntimeError, match="larger than the file"):
        moe.Gguf(str(p))
    # cut inside the tensor data, then inside the header
    gw.write_gguf(tmp_path / "ok.gguf", _meta(), _tensors(rng))
    full = (tmp_path / "ok.gguf").read_bytes()
    (tmp_path / "cut.gguf").write_bytes(full[:-100])
    with pytest.raises(RuntimeError, match="past the end"):
        moe.Gguf(str(tmp_path / "cut.gguf"))
    (tmp_path / "cut2.gguf").write_bytes(full[:60])
    with pytest.raises(RuntimeError, match="truncated"):
        moe.Gguf(str(tmp_path / "cut2.gguf"))
    with pytest.raises(RuntimeError, match="cannot open"):
        moe.Gguf(str(tmp_path / "nothing.gguf"))


def test_type_info():
    b, n = C.c_int(), C.c_int()
    for t, want in ((12, (256, 144)), (8, (32, 34)), (9, (32, 36)), (0, (1, 4)), (13, (256, 176)), (7, (32, 24))):
        check(lib().sfnx_gguf_type_info(t, C.byref(b), C.byref(n)))
        assert (b.value, n.value) == want
    assert lib().sfnx_gguf_type_info(99, None, None) != 0
