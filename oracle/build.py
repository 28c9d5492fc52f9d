"""Build the oracle (test infrastructure) as oracle/liboracle_kurumi.so with g++.

The oracle links the product library only for the IR data structures (graph/tensor
handles); the product never links the oracle. The reference itself (Rust) cannot be built in
this image, so there is no oracle/_ref build.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
LIB = HERE / "liboracle_kurumi.so"
PKG = ROOT / "kurumi_amd"

FLAGS = ["-std=c++17", "-O3", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
         "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{ROOT}"]


def build(verbose: bool = False) -> Path:
    srcs = sorted(str(p) for p in HERE.glob("*.cpp"))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["g++", *FLAGS, *srcs, "-o", str(tmp), f"-L{PKG}", "-lkurumi_hip", "-Wl,-rpath,$ORIGIN/../kurumi_amd"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    tmp.replace(LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
