"""GPU tests of the profile step: wtc_profile_tiles times one variant, and
wtc-compiler --enable-profiling ranks the solver's first candidates by their
measured time, writes profiledMs, and plans the launch with the fastest."""
from __future__ import annotations

import ctypes
import json
import subprocess
from pathlib import Path

import pytest

torch = pytest.importorskip("torch")

from welder_typical_chain_amd.chain_mlir import chain_mlir  # noqa: E402
from welder_typical_chain_amd.configs import CONFIGS  # noqa: E402

pytestmark = pytest.mark.gpu

needs_gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="no GPU")
CLI = Path(__file__).resolve().parents[1] / "welder_typical_chain_amd" / "wtc-compiler"


@needs_gpu
def test_profile_tiles_times_a_variant(native_lib):
    from welder_typical_chain_amd import _lib
    print("\n[gpu-case] wtc_profile_tiles C2 on two variants", flush=True)
    us = ctypes.c_double()
    for tiles in ([128, 128, 64, 2, 32], [128, 128, 64, 2, 16]):
        t = _lib.Tiles(*tiles)
        rc = _lib.lib().wtc_profile_tiles(1, 2048, 2048, 1024, _lib.DTYPE_F16, _lib.DTYPE_F16,
                                          ctypes.byref(t), _lib.PATH_EXCHANGE, 5, 50, 1,
                                          ctypes.byref(us))
        _lib.check(rc)
        print(f"[gpu-case] {tiles}: {us.value:.2f} us per call", flush=True)
        assert 5.0 < us.value < 200.0
    t = _lib.Tiles(256, 128, 64, 2, 32)  # no exchange path on the 256-row variant
    rc = _lib.lib().wtc_profile_tiles(1, 2048, 2048, 1024, _lib.DTYPE_F16, _lib.DTYPE_F16,
                                      ctypes.byref(t), _lib.PATH_EXCHANGE, 1, 1, 1, ctypes.byref(us))
    assert rc == _lib.WTC_ERR_UNSUPPORTED


@needs_gpu
def test_wtc_compiler_profiles_the_top_candidates(native_lib, tmp_path):
    src = tmp_path / "c2.mlir"
    src.write_text(chain_mlir(CONFIGS["C2"]))
    out = tmp_path / "out"
    print("\n[gpu-case] wtc-compiler --enable-profiling on C2, top 3", flush=True)
    r = subprocess.run([str(CLI), "--input", str(src), "--output-dir", str(out), "--enable-profiling",
                        "--profile-top-k", "3", "--profile-iters", "100"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    print((out / "search" / "profile.log").read_text(), flush=True)
    rows = [line.split("\t") for line in
            (out / "search" / "candidates.tsv").read_text().strip().split("\n")[1:]]
    profiled = [float(row[8]) for row in rows]
    assert all(p > 0 for p in profiled[:3]) and all(p < 0 for p in profiled[3:])
    assert profiled[:3] == sorted(profiled[:3])
    best = json.loads((out / "search" / "best.json").read_text())
    top = [int(v) for v in rows[0][1:6]]
    assert [best[k] for k in ("tileM", "tileN", "tileK", "threadTileM", "threadTileN")] == top
    launch = json.loads((out / "fused" / "05.out.hip.launch.json").read_text())
    assert [launch["tiles"][k] for k in ("tileM", "tileN", "tileK", "threadTileM",
                                         "threadTileN")] == top
