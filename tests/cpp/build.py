"""Builds the C++ integration programs of tests/cpp (host code over libsfnx_moe.so) in place."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
PROGRAMS = ["moe_window"]


def build(verbose: bool = False) -> None:
    for name in PROGRAMS:
        cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-O2", f"-I{ROOT / 'include'}", f"-I{ROOT / 'sfnx_amd' / 'include'}",
               str(HERE / f"{name}.cpp"), f"-L{ROOT / 'sfnx_amd'}", "-lsfnx_moe", "-Wl,-rpath,$ORIGIN/../../sfnx_amd",
               "-o", str(HERE / name)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"building {name} failed:\n{r.stderr}")
        if verbose:
            print(f"built {HERE / name}")


if __name__ == "__main__":
    build(verbose=True)
