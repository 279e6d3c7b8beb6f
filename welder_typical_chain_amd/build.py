"""Builds the native parts of the package in-tree.

- ``libwtc_hip.so``: the gfx950 HIP kernels plus the C-ABI (launcher, and the
  reference's compile / solver entry points), compiled with hipcc.
- ``libwelder-compile-capi.so`` (a link to ``libwtc_hip.so``) and
  ``libwelder-solver-capi.so`` (CPU only: chain recogniser + tile solver): the
  file names the reference's toolchain looks for in its backend build
  directory (reference compiler/backend/Toolchain.cpp:29-45).
- ``libwtc_hip_stamps.so``: the same library with the exchange kernel's
  phase stamps compiled in (``-DWTC_PHASE_STAMPS``), for
  ``python -m welder_typical_chain_amd.phase_timeline``; never loaded by the
  product path.
- ``wtc-compiler``: the reference's pipeline driver CLI (``--search-only``,
  ``--compile-only``, full) over the two C-ABIs, linked against
  ``libwtc_hip.so`` next to it.
- ``<source>.gfx950.co``: the device code object of each HIP source, and
  ``kernel_resources.json``: per kernel, the register / LDS / scratch figures
  from the code object's metadata and instruction counts (MFMA, LDS DMA,
  scratch) from its disassembly.  The compile C-ABI reports them.

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
STAMPS_LIB = PKG / "libwtc_hip_stamps.so"
STAMPS_SRC = "fused_matmul_softmax.hip"
COMPILE_LIB = PKG / "libwelder-compile-capi.so"
SOLVER_LIB = PKG / "libwelder-solver-capi.so"
CLI = PKG / "wtc-compiler"
RESOURCES = PKG / "kernel_resources.json"
BUILD_INFO = PKG / "build_info.json"
RESOURCES_TSV = PKG / "kernel_resources.tsv"
TSV_COLUMNS = ["vgpr_count", "agpr_count", "sgpr_count", "vgpr_spill_count", "sgpr_spill_count",
               "lds_bytes", "scratch_bytes", "mfma", "lds_dma_loads", "ds_read_tr", "scratch_ops",
               "instructions"]
LLVM_BIN = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "llvm" / "bin"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["fused_matmul_softmax.hip", "wide_tile.hip", "rowblock_softmax.hip", "unfused_chain.hip",
               "launch.hip"]
CXX_SOURCES = ["chain_recognizer.cpp", "variants.cpp", "tile_solver.cpp", "compile_capi.cpp"]

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
# Per-source extra flags.  The tile kernels take their first-load scalars as
# leading arguments; gfx950 preloads those into SGPRs.
HIP_EXTRA = {"fused_matmul_softmax.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
             "wide_tile.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"]}
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
        _run([HIPCC, *HIP_FLAGS, *HIP_EXTRA.get(src, []), "-c", str(path), "-o", str(obj)])
    else:
        _run(["g++", *CXX_FLAGS, "-c", str(path), "-o", str(obj)])
    return obj


def _compile_stamps() -> Path:
    obj = OBJ / (STAMPS_SRC + ".stamps.o")
    _run([HIPCC, *HIP_FLAGS, *HIP_EXTRA.get(STAMPS_SRC, []), "-DWTC_PHASE_STAMPS", "-c",
          str(CSRC / STAMPS_SRC), "-o", str(obj)])
    return obj


def _code_object(src: str) -> Path:
    """Device code object of one HIP source (same flags as the library)."""
    bundle = OBJ / (src + ".bundle")
    co = PKG / (Path(src).stem + f".{ARCH}.co")
    _run([HIPCC, *HIP_FLAGS, *HIP_EXTRA.get(src, []), "--genco", str(CSRC / src), "-o", str(bundle)])
    _run([str(LLVM_BIN / "clang-offload-bundler"), "--unbundle", "--type=o",
          f"--targets=hipv4-amdgcn-amd-amdhsa--{ARCH}", f"--input={bundle}", f"--output={co}"])
    return co


def _kernel_resources(code_objects: list[Path]) -> dict:
    """Per-kernel metadata and instruction counts of our own code objects."""
    import yaml

    kernels = {}
    for co in code_objects:
        notes = subprocess.run([str(LLVM_BIN / "llvm-readelf"), "--notes", str(co)],
                               capture_output=True, text=True, check=True).stdout
        start = notes.find("---")
        end = notes.find("...", start)
        meta = yaml.safe_load(notes[start:end]) if start >= 0 else {}
        for k in meta.get("amdhsa.kernels", []):
            kernels[k[".name"]] = {
                "code_object": co.name,
                "vgpr_count": k.get(".vgpr_count"), "agpr_count": k.get(".agpr_count"),
                "sgpr_count": k.get(".sgpr_count"),
                "vgpr_spill_count": k.get(".vgpr_spill_count"),
                "sgpr_spill_count": k.get(".sgpr_spill_count"),
                "lds_bytes": k.get(".group_segment_fixed_size"),
                "scratch_bytes": k.get(".private_segment_fixed_size"),
                "max_flat_workgroup_size": k.get(".max_flat_workgroup_size"),
            }
        dis = subprocess.run([str(LLVM_BIN / "llvm-objdump"), "-d", "--no-show-raw-insn", str(co)],
                             capture_output=True, text=True, check=True).stdout
        cur = None
        for line in dis.splitlines():
            if line.endswith(">:") and "<" in line:
                cur = kernels.get(line[line.index("<") + 1:-2])
                if cur is not None:
                    cur.update(mfma=0, lds_dma_loads=0, ds_read_tr=0, scratch_ops=0, instructions=0)
                continue
            if cur is None or not line.startswith("\t"):
                continue
            insn = line.split("//")[0].split()
            if not insn:
                continue
            op = insn[0]
            cur["instructions"] += 1
            if op.startswith("v_mfma"):
                cur["mfma"] += 1
            elif op.startswith("buffer_load") and insn[-1] == "lds":
                cur["lds_dma_loads"] += 1
            elif op.startswith("ds_read_b64_tr"):
                cur["ds_read_tr"] += 1
            elif op.startswith("scratch_"):
                cur["scratch_ops"] += 1
    return {"target": ARCH, "kernels": kernels}


def source_digest() -> str:
    """SHA-256 over the sources a build compiles (csrc/ and include/wtc/),
    in name order: the stamp that ties a measurement to the build it ran."""
    import hashlib
    h = hashlib.sha256()
    files = sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp"), *CSRC.glob("*.h"),
                    *(ROOT / "include" / "wtc").glob("*.h")])
    for f in files:
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()[:16]


def _write_build_info() -> None:
    import json
    info = {"source_digest": source_digest()}
    try:
        head = subprocess.run(["git", "-C", str(ROOT), "rev-parse", "--short", "HEAD"],
                              capture_output=True, text=True, timeout=10)
        dirty = subprocess.run(["git", "-C", str(ROOT), "status", "--porcelain", "--", "include",
                                str(CSRC)], capture_output=True, text=True, timeout=10)
        if head.returncode == 0:
            info["git_head"] = head.stdout.strip()
            info["sources_changed_since_head"] = bool(dirty.stdout.strip())
    except (OSError, subprocess.SubprocessError):
        pass
    BUILD_INFO.write_text(json.dumps(info, indent=1) + "\n")


def build_info() -> dict:
    """The stamp of the library in this tree ({} if it was never built)."""
    import json
    try:
        return json.loads(BUILD_INFO.read_text())
    except (OSError, ValueError):
        return {}


def build(verbose: bool = False) -> Path:
    """Compile every source (always; no staleness shortcut) and link."""
    import json

    OBJ.mkdir(exist_ok=True)
    sources = HIP_SOURCES + [s for s in CXX_SOURCES if (CSRC / s).exists()]
    device_only = [s for s in HIP_SOURCES if s != "launch.hip"]
    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        co_jobs = [ex.submit(_code_object, s) for s in device_only]
        stamps_job = ex.submit(_compile_stamps)
        objs = list(ex.map(_compile_one, sources))
        code_objects = [j.result() for j in co_jobs]
        stamps_obj = stamps_job.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    stamps_objs = [stamps_obj if o.name == STAMPS_SRC + ".o" else o for o in objs]
    tmp = STAMPS_LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, stamps_objs)])
    os.replace(tmp, STAMPS_LIB)
    if COMPILE_LIB.is_symlink() or COMPILE_LIB.exists():
        COMPILE_LIB.unlink()
    COMPILE_LIB.symlink_to(LIB.name)
    cpu_objs = [str(OBJ / (s + ".o")) for s in ("chain_recognizer.cpp", "variants.cpp", "tile_solver.cpp")]
    tmp = SOLVER_LIB.with_suffix(".so.tmp")
    _run(["g++", "-shared", "-Wl,--no-undefined", "-o", str(tmp), *cpu_objs])
    os.replace(tmp, SOLVER_LIB)
    rocm_lib = str(Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "lib")
    tmp = CLI.with_suffix(".tmp")
    _run(["g++", *CXX_FLAGS, str(CSRC / "wtc_compiler.cpp"), "-o", str(tmp), f"-L{PKG}", "-lwtc_hip",
          f"-Wl,-rpath-link,{rocm_lib}", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, CLI)
    res = _kernel_resources(code_objects)
    RESOURCES.write_text(json.dumps(res, indent=1, sort_keys=True) + "\n")
    # the same figures as a flat table for the compile C-ABI's report
    rows = ["\t".join(["kernel", "code_object", *TSV_COLUMNS])]
    for name, k in sorted(res["kernels"].items()):
        rows.append("\t".join([name, k["code_object"], *(str(k.get(c, 0)) for c in TSV_COLUMNS)]))
    RESOURCES_TSV.write_text("\n".join(rows) + "\n")
    _write_build_info()
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
