"""CPU tests of the wtc-compiler CLI: the reference's pipeline driver modes
(compiler/main.cpp:10-90, compiler/pipeline/PipelineRunner.cpp:52-219) over
this library's recogniser, solver and compile C-ABIs.  Nothing here launches
a kernel."""
from __future__ import annotations

import json
import subprocess
from pathlib import Path

import pytest

from welder_typical_chain_amd.chain_mlir import chain_mlir
from welder_typical_chain_amd.configs import CONFIGS

ROOT = Path(__file__).resolve().parents[1]
CLI = ROOT / "welder_typical_chain_amd" / "wtc-compiler"
REF_MLIR = Path("/root/reference/mlir")


@pytest.fixture(scope="module")
def cli(native_lib):
    if not CLI.exists():
        from welder_typical_chain_amd import build
        build.build()
    return CLI


def run(cli, *args):
    return subprocess.run([str(cli), *map(str, args)], capture_output=True, text=True, timeout=60)


@pytest.fixture()
def c2_mlir(tmp_path):
    p = tmp_path / "c2.mlir"
    p.write_text(chain_mlir(CONFIGS["C2"]))
    return p


def test_full_mode_layout(cli, c2_mlir, tmp_path):
    out = tmp_path / "out"
    r = run(cli, "--input", c2_mlir, "--output-dir", out, "--verbose")
    assert r.returncode == 0, r.stderr
    assert "[wtc-compiler] done: " in r.stdout
    for rel in ["ir/01.canonicalized.mlir", "ir/01.canonicalize.log", "ir/02.tagged.mlir",
                "ir/02.tags.json", "search/best.json", "search/best_summary.json",
                "search/candidates.tsv", "search/solver.log", "fused/03.chain.canonical.mlir",
                "fused/04.kernel.plan.json", "fused/05.out.hip.launch.json",
                "fused/kernel_report.txt", "fused/compile.log", "fused/postbufferize_report.txt"]:
        assert (out / rel).is_file() and (out / rel).stat().st_size > 0, rel
    tags = json.loads((out / "ir" / "02.tags.json").read_text())
    assert tags["pipeline"] == "typical_chain" and tags["counts"]["matmul"] == 1
    assert tags["problem"]["m"] == 2048 and tags["problem"]["k"] == 1024
    tagged = (out / "ir" / "02.tagged.mlir").read_text()
    assert tagged.startswith("// [wtc tagging]") and "// wtc.tag: welder.matmul_anchor" in tagged
    best = json.loads((out / "search" / "best.json").read_text())
    assert set(best) == {"tileM", "tileN", "tileK", "threadTileM", "threadTileN"}
    launch = json.loads((out / "fused" / "05.out.hip.launch.json").read_text())
    assert launch["path"] == "exchange" and launch["problem"]["m"] == 2048
    report = dict(l.split("=", 1) for l in
                  (out / "fused" / "postbufferize_report.txt").read_text().splitlines())
    assert report["post_matmul_count"] == "1" and report["launch_kernel_count"] == "1"
    assert int(report["mfma_instruction_count"]) > 0 and report["vgpr_spill_count"] == "0"


def test_search_only_stops_after_best_json(cli, c2_mlir, tmp_path):
    out = tmp_path / "out"
    r = run(cli, "--input", c2_mlir, "--output-dir", out, "--search-only")
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == f"[wtc-compiler] tiles written to {out / 'search' / 'best.json'}"
    assert (out / "search" / "candidates.tsv").is_file()
    assert not (out / "fused").exists()


def test_compile_only_with_best_json_skips_search(cli, c2_mlir, tmp_path):
    first = tmp_path / "first"
    assert run(cli, "--input", c2_mlir, "--output-dir", first, "--search-only").returncode == 0
    out = tmp_path / "out"
    r = run(cli, "--input", c2_mlir, "--output-dir", out, "--compile-only",
            "--best-json", first / "search" / "best.json")
    assert r.returncode == 0, r.stderr
    assert not (out / "search" / "candidates.tsv").exists()  # no solver run
    assert (out / "search" / "best.json").read_text() == (first / "search" / "best.json").read_text()
    assert (out / "fused" / "05.out.hip.launch.json").is_file()


def test_baseline_mode_compiles_unfused(cli, c2_mlir, tmp_path):
    out = tmp_path / "out"
    r = run(cli, "--input", c2_mlir, "--output-dir", out, "--baseline")
    assert r.returncode == 0, r.stderr
    plan = json.loads((out / "baseline" / "04.kernel.plan.json").read_text())
    assert plan["path"] == "unfused" and len(plan["kernels"]) == 5 and plan["fused"] is False


def test_no_search_and_tile_overrides(cli, c2_mlir, tmp_path):
    out = tmp_path / "out"
    r = run(cli, "--input", c2_mlir, "--output-dir", out, "--no-search", "--verbose")
    assert r.returncode == 0, r.stderr
    assert "default variant of the input type" in r.stdout
    # an override that no kernel variant implements fails at compile, with the
    # available variants named
    r = run(cli, "--input", c2_mlir, "--output-dir", tmp_path / "o2", "--tile-m", "48")
    assert r.returncode == 1 and "no gfx950 kernel variant implements" in r.stderr
    best = json.loads((tmp_path / "o2" / "search" / "best.json").read_text())
    assert best["tileM"] == 48


def test_repeat_writes_iteration_dirs(cli, c2_mlir, tmp_path):
    out = tmp_path / "out"
    r = run(cli, "--input", c2_mlir, "--output-dir", out, "--repeat", "3")
    assert r.returncode == 0, r.stderr
    for i in range(3):
        assert (out / f"iter_{i}" / "fused" / "05.out.hip.launch.json").is_file()


def test_named_softmax_and_batched_inputs(cli, tmp_path):
    for name, kw in [("named", dict(named_softmax=True)), ("batched", dict(batch=4))]:
        src = tmp_path / f"{name}.mlir"
        src.write_text(chain_mlir(CONFIGS["C3"] if name == "batched" else CONFIGS["C2"], **kw))
        out = tmp_path / name
        r = run(cli, "--input", src, "--output-dir", out)
        assert r.returncode == 0, (name, r.stderr)
        canonical = (out / "ir" / "01.canonicalized.mlir").read_text()
        assert "linalg.softmax" not in canonical and "math.exp" in canonical


def test_argument_errors(cli, c2_mlir, tmp_path):
    assert run(cli).returncode == 2                                   # --input missing
    assert run(cli, "--input", c2_mlir, "--bogus").returncode == 2      # unknown argument
    assert run(cli, "--input", c2_mlir, "--repeat", "0").returncode == 2
    assert run(cli, "--input", c2_mlir, "--backend-mode", "x").returncode == 2
    assert run(cli, "--input", c2_mlir, "--tile-m", "x").returncode == 2
    assert run(cli, "--help").returncode == 0
    r = run(cli, "--input", tmp_path / "missing.mlir", "--output-dir", tmp_path / "o")
    assert r.returncode == 1 and "not a Matmul -> row-Softmax chain" in r.stderr
    bad = tmp_path / "bad.mlir"
    bad.write_text("func.func @f() { return }\n")
    r = run(cli, "--input", bad, "--output-dir", tmp_path / "o2")
    assert r.returncode == 1 and "chain not recognised" in r.stderr
    assert (tmp_path / "o2" / "ir" / "01.canonicalize.log").is_file()


@pytest.mark.skipif(not REF_MLIR.exists(), reason="reference chain files not present")
@pytest.mark.parametrize("fname", ["matmul_softmax_chain.mlir", "matmul_softmax_chain_f16_native.mlir",
                                   "matmul_softmax_chain_named_softmax.mlir"])
def test_reference_chain_files_full_pipeline(cli, tmp_path, fname):
    out = tmp_path / "out"
    r = run(cli, "--input", REF_MLIR / fname, "--output-dir", out)
    assert r.returncode == 0, r.stderr
    assert (out / "fused" / "postbufferize_report.txt").is_file()


def test_profiling_without_a_gpu_keeps_the_model_ranking(cli, c2_mlir, tmp_path):
    """--enable-profiling on a host without a GPU: the first measurement
    fails, the log says so, and the model's ranking and best.json stand."""
    ref = tmp_path / "ref"
    assert run(cli, "--input", c2_mlir, "--output-dir", ref, "--search-only").returncode == 0
    out = tmp_path / "prof"
    r = run(cli, "--input", c2_mlir, "--output-dir", out, "--search-only", "--enable-profiling",
            "--profile-top-k", "2", "--profile-iters", "5")
    assert r.returncode == 0, r.stderr
    log = (out / "search" / "profile.log").read_text()
    assert "rc=" in log and "model ranking kept" in log
    assert (out / "search" / "best.json").read_text() == (ref / "search" / "best.json").read_text()
    assert (out / "search" / "candidates.tsv").read_text() == \
        (ref / "search" / "candidates.tsv").read_text()
    bad = run(cli, "--input", c2_mlir, "--output-dir", out, "--profile-iters", "0")
    assert bad.returncode == 2 and "positive integer" in bad.stderr
