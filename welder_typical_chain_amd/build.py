"""Builds the native parts of the package in-tree.

- ``libwtc_hip.so``: the gfx950 HIP kernels plus the C-ABI (launcher, and the
  reference's compile / solver entry points), compiled with hipcc.
- ``wtc-compiler``: the CLI front end (C++17, g++), which dlopens the library
  exactly as the reference's CLI dlopens its backend libraries.

Everything lands next to this file so the built artefacts travel with the
source tree.  Run ``python -m welder_typical_chain_amd.build``.
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
OBJ = PKG / "_build"
LIB = PKG / "libwtc_hip.so"
CLI = PKG / "wtc-compiler"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["fused_matmul_softmax.hip", "unfused_chain.hip", "launch.hip"]
CXX_SOURCES = ["chain_recognizer.cpp", "tile_solver.cpp", "compile_capi.cpp"]

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # packed fp32 VALU forms are kept out of the generated code on purpose
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra",
             f"-I{ROOT / 'include'}", f"-I{CSRC}"]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{err}")


def _compile_one(src: str) -> Path:
    path = CSRC / src
    obj = OBJ / (src + ".o")
    if path.suffix == ".hip":
        _run([HIPCC, *HIP_FLAGS, "-c", str(path), "-o", str(obj)])
    else:
        _run(["g++", *CXX_FLAGS, "-c", str(path), "-o", str(obj)])
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source (always; no staleness shortcut) and link."""
    OBJ.mkdir(exist_ok=True)
    sources = HIP_SOURCES + [s for s in CXX_SOURCES if (CSRC / s).exists()]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile_one, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    cli_src = CSRC / "wtc_compiler_main.cpp"
    if cli_src.exists():
        _run(["g++", *CXX_FLAGS, "-o", str(CLI), str(cli_src),
              *[str(o) for o in objs if o.name.endswith(".cpp.o")], "-ldl"])
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
