"""The C-ABI library: it loads, exports every symbol include/sfnx_moe.h declares, and rejects bad arguments with a
status and a message before touching the GPU (src/kernels.cu:31-34 and src/moe.cuh:473-494 throw on the same)."""
import ctypes as C
from pathlib import Path

import pytest

from sfnx_amd import _abi


def test_library_exports_every_declared_symbol():
    lib = _abi.lib()
    declared = _abi.declared_symbols()
    assert len(declared) >= 18
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_abi.SIGNATURES), "bindings and header disagree"
    assert lib.sfnx_abi_version() == 1


def test_row_bytes():
    lib = _abi.lib()
    assert lib.sfnx_row_bytes(_abi.Q4_K, 2048) == 1152
    assert lib.sfnx_row_bytes(_abi.Q4_K, 512) == 288
    assert lib.sfnx_row_bytes(_abi.Q8_0, 2048) == 2176


# a host sfnx_q8s whose (never dereferenced) device pointers are non-null: the calls below fail their checks first
_Q8S = _abi.Q8S(1, 1)
_Q8S_PTR = C.addressof(_Q8S)


@pytest.mark.parametrize("call, msg", [
    (lambda L: L.sfnx_router_route(None, None, None, 0, 2048, 512, 10, None, None, None, None, None, 1, None), "T out of range"),
    (lambda L: L.sfnx_router_route(None, None, None, 17, 2048, 512, 10, None, None, None, None, None, 1, None), "T out of range"),
    (lambda L: L.sfnx_router_route(None, None, None, 1, 2048, 500, 10, None, None, None, None, None, 1, None), "E must be"),
    (lambda L: L.sfnx_router_route(None, None, None, 1, 2048, 512, 17, None, None, None, None, None, 1, None), "K out of range"),
    (lambda L: L.sfnx_router_route_plan(None, None, None, 1, 2048, 512, 10, None, None, None, None, None, 0, None, 0, None,
                                        None), "null list"),
    (lambda L: L.sfnx_router_route_plan(None, None, None, 1, 2048, 512, 10, None, None, None, None, None, 0, None, 0,
                                        C.c_void_p(8), None), "null expert cache"),
    (lambda L: L.sfnx_moe_gate_up(None, 1 << 30, 5, 2048, 1024, None, None, 11, 1, None, None, None), "Q4_K (12) or Q5_K (13)"),
    (lambda L: L.sfnx_moe_gate_up(None, 1 << 30, 12, 2000, 1024, None, None, 11, 1, None, None, None), "multiple of 512"),
    (lambda L: L.sfnx_moe_gate_up(None, 1000, 12, 2048, 1024, None, None, 11, 1, None, None, None), "stride smaller"),
    (lambda L: L.sfnx_moe_down(None, 1 << 30, 12, 512, 2048, None, None, 11, 0, None, None, None), "T out of range"),
    (lambda L: L.sfnx_store_pack(12, None, None, 1, 4, 256, None), "multiple of 512"),
    (lambda L: L.sfnx_quantize_q8_1(None, None, 30, 1, None), "multiple of 32"),
    (lambda L: L.sfnx_pf_route(None, 0, 512, 10, None, None, None, None, None, None, None, 1, None), "C must be positive"),
    (lambda L: L.sfnx_q8s_gemv(_Q8S_PTR, 100, 2048, 1, 1, 100, 1, None), "rows must be"),
    (lambda L: L.sfnx_q8s_gemv(_Q8S_PTR, 96, 2000, 1, 1, 96, 1, None), "cols must be"),
    (lambda L: L.sfnx_q8s_gemv(_Q8S_PTR, 96, 2048, 1, 1, 64, 1, None), "out_stride"),
    (lambda L: L.sfnx_q8s_gemv(None, 96, 2048, 1, 1, 96, 1, None), "null pointer"),
    (lambda L: L.sfnx_q8s_split(1, 96, 2000, _Q8S_PTR, None), "multiple of 32"),
    (lambda L: L.sfnx_swiglu_stacked_q8_1(1, 1, 500, 1, None), "ffs must be"),
    (lambda L: L.sfnx_pf_dense(_Q8S_PTR, 1024, 2000, 1, 10, 1, 1024, 1, 1 << 30, None), "cols of 512"),
    (lambda L: L.sfnx_pf_dense(_Q8S_PTR, 1000, 2048, 1, 10, 1, 1024, 1, 100, None), "multiple of 256"),
    (lambda L: L.sfnx_pf_dense(_Q8S_PTR, 1024, 2048, 1, 10, 1, 1024, 1, 100, None), "wk smaller"),
    (lambda L: L.sfnx_hc_read(1, None, None, 1, 1, 1, 1, 1, None, 1e-6, 1, None, None, 1, 2000, 4, 320, 1, 1 << 30, None), "N must be"),
    (lambda L: L.sfnx_hc_read(1, None, None, 1, 1, 1, 1, 1, None, 1e-6, 1, None, None, 1, 2560, 9, 320, 1, 1 << 30, None), "HC must be"),
    (lambda L: L.sfnx_hc_read(1, None, None, 1, 1, 1, 1, 1, None, 1e-6, 1, None, None, 1, 2560, 4, 330, 1, 1 << 30, None), "LR must be"),
    (lambda L: L.sfnx_hc_read(1, None, None, 1, 1, 1, 1, 1, None, 1e-6, 1, None, None, 1, 2560, 8, 512, 1, 1 << 30, None), "HC LR must be"),
    (lambda L: L.sfnx_hc_read(1, None, None, 1, 1, 1, 1, 1, None, 1e-6, 1, None, None, 1, 2560, 4, 320, 1, 10, None), "workspace smaller"),
    (lambda L: L.sfnx_hc_read(1, 1, None, 1, 1, 1, 1, 1, None, 1e-6, 1, None, None, 1, 2560, 4, 320, 1, 1 << 30, None), "inj_prev"),
    (lambda L: L.sfnx_moe_decode_q8s(1, None, 1, 12, 12, 2048, 512, 10, 512, 1, 1, 1, 1e-6, 1, 1 << 30, 0, None), "no shared expert"),
])
def test_bad_arguments_are_refused(call, msg):
    lib = _abi.lib()
    assert call(lib) == -1
    assert msg in lib.sfnx_last_error().decode()


def test_cpp_header_compiles():
    """the C++ mirror of the reference's entry points compiles against the C header (host only)"""
    import subprocess
    import tempfile
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    src = ('#include "sfnx/kernels.hpp"\n#include "sfnx/gguf.hpp"\n'
           'int main() { return sizeof(sfnx::Job) == 136 && sizeof(sfnx::BigJob) == 520 ? 0 : 1; }\n')
    with tempfile.TemporaryDirectory() as d:
        f = Path(d) / "t.cpp"
        f.write_text(src)
        r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", f"-I{root / 'sfnx_amd' / 'include'}",
                            f"-I{root / 'include'}", "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__", str(f)],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


def test_expert_cache_struct_layout_matches_the_header(tmp_path):
    """the ctypes mirror of sfnx_expert_cache has the C compiler's size and field offsets"""
    import ctypes as C
    import subprocess
    fields = [f[0] for f in _abi.ExpertCacheC._fields_]
    src = tmp_path / "ec.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "sfnx_moe.h"\nint main(void) {\n'
                   '  printf("%zu\\n", sizeof(sfnx_expert_cache));\n' +
                   "".join(f'  printf("%zu\\n", offsetof(sfnx_expert_cache, {f}));\n' for f in fields) + "  return 0;\n}\n")
    exe = tmp_path / "ec"
    inc = Path(__file__).resolve().parents[1] / "include"
    subprocess.run(["gcc", "-std=c99", "-I", str(inc), str(src), "-o", str(exe)], check=True)
    out = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert out[0] == C.sizeof(_abi.ExpertCacheC)
    assert out[1:] == [getattr(_abi.ExpertCacheC, f).offset for f in fields]


def test_router_plan_refuses_tables_without_the_shared_expert():
    """a cache whose tables hold only the E routed experts a layer cannot plan a window with the shared job (expert E);
    refused on the host, before any launch"""
    c = _abi.ExpertCacheC()
    c.n_slots, c.n_pools, c.n_layers, c.n_experts = 8, 1, 1, 64
    c.s0[0], c.n[0], c.slot_bytes[0], c.dn_off[0], c.pool[0] = 0, 8, 32, 16, 16
    c.ep_gu = c.ep_dn = c.host_gu = c.host_dn = c.slot_of = c.owner = c.ref = c.hand = 16
    L = _abi.lib()
    args = (None, None, None, 1, 1024, 64, 6, None, None, None, None, None)
    assert L.sfnx_router_route_plan(*args, 1, C.byref(c), 0, C.c_void_p(16), None) != 0
    assert "pass the cache's tables" in L.sfnx_last_error().decode()
