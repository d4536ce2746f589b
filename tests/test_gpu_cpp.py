"""The C++ face (sfnx/kernels.hpp) from a C++ host program, as the reference engine would call it: a decode window
through the unfused calls (with the shared expert as expert E, and as dense Q8_0 through router_route's and
moe_gate_up's shared-expert arguments) against the fused decode, bit for bit; a prompt chunk through the prompt
path's calls; and decode windows through an ExpertCache (router_route's plan, moe_cache, DW::ep tables) against the
resident store, bit for bit (tests/cpp/moe_window.cpp)."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
PROG = Path(__file__).resolve().parent / "cpp" / "moe_window"


def test_cpp_decode_window():
    if not PROG.exists():
        from tests.cpp import build
        build.build()
    r = subprocess.run([str(PROG)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok")
