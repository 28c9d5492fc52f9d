"""Build libkurumi_hip.so in-tree: host C++ with g++, HIP kernels with hipcc for gfx950.

Run as ``python -m kurumi_amd.build`` (or through ``__graft_entry__.build()``). Objects go to
``kurumi_amd/_build/``; the library lands next to this file so it travels with the tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libkurumi_hip.so"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HOST_FLAGS = ["-std=c++17", "-O2", "-fPIC", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{ROOT / 'include'}",
              "-Wall", "-Wno-unused-function", "-Wno-sign-compare"]
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", f"-I{ROOT / 'include'}", "-Wno-unused-command-line-argument"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def sources() -> tuple[list[Path], list[Path]]:
    host = sorted(CSRC.glob("ir/*.cpp")) + sorted(CSRC.glob("hip/*.cpp")) + sorted(CSRC.glob("capi/*.cpp"))
    dev = sorted(CSRC.glob("hip/kernels/*.hip"))
    return host, dev


def _up_to_date(o: Path) -> bool:
    """True when `o` and its dependency file exist and no listed dependency is newer."""
    d = o.with_suffix(".d")
    if not o.exists() or not d.exists():
        return False
    deps = d.read_text().replace("\\\n", " ").split(":", 1)[-1].split()
    t = o.stat().st_mtime
    try:
        return all(Path(p).stat().st_mtime <= t for p in deps)
    except FileNotFoundError:
        return False


def build(verbose: bool = False, jobs: int | None = None, incremental: bool = False) -> Path:
    """Compile every source (or, with `incremental`, those whose dependencies changed) and link."""
    BUILD.mkdir(exist_ok=True)
    host, dev = sources()
    cmds = []
    objs = []
    for s in host:
        o = BUILD / (s.parent.name + "_" + s.stem + ".o")
        if not (incremental and _up_to_date(o)):
            cmds.append(["g++", *HOST_FLAGS, "-MMD", "-MF", str(o.with_suffix(".d")), "-c", str(s), "-o", str(o)])
        objs.append(o)
    for s in dev:
        o = BUILD / ("k_" + s.stem + ".o")
        if not (incremental and _up_to_date(o)):
            cmds.append([f"{ROCM}/bin/hipcc", *HIP_FLAGS, "-MMD", "-MF", str(o.with_suffix(".d")), "-c", str(s), "-o",
                         str(o)])
        objs.append(o)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, c) for c in cmds]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([f"{ROCM}/bin/hipcc", "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          f"-L{ROCM}/lib", "-lhiprtc", "-lamdhip64", "-pthread", f"-Wl,-rpath,{ROCM}/lib",
          # calls and function addresses inside the library bind to its own definitions, so a
          # process that also loads kurumi's library (same ku_* names) cannot divert them
          "-Wl,-Bsymbolic-functions"])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv)
    sys.exit(0)
