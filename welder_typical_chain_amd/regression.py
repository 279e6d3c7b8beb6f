"""Artefact regression run of the wtc-compiler command line.

The counterpart of the reference's bench/run_regression.sh:1-115, with the
same four runs and the same file names and patterns:

1. ``search_api``: ``--search-only`` writes ``search/best.json`` and
   ``search/candidates.tsv`` (run_regression.sh:58-69);
2. ``named_softmax``: ``--search-only`` on a chain with a named
   ``linalg.softmax`` leaves a canonical chain with ``math.exp`` and
   ``arith.divf`` and no ``linalg.softmax`` (run_regression.sh:71-86);
3. ``full_api_default``: the full ``--fused`` pipeline writes
   ``05.out.nvvm.runnable.mlir`` with a ``gpu.launch_func`` per kernel, and
   ``04.after_workgroup_launch.mlir`` whose launches carry their LDS as a
   ``workgroup(...)`` attribution (run_regression.sh:88-98);
4. ``pure_api_repeat``: ``--pure-api-full --fused --repeat N`` writes the
   same runnable module into ``iter_<N-1>`` (run_regression.sh:100-112).

Each check appends ``check  status  detail`` to ``regression_summary.tsv``;
the first failure ends the run with status 1.  With no ``--input`` the runs
use a generated chain of the reference's default input
(mlir/matmul_softmax_chain_f16_native.mlir:7: f16 8192x64 . 64x128, f32 out)
and its named-softmax twin.

Usage: ``python -m welder_typical_chain_amd.regression [--out-base D]
[--input F] [--named-softmax-input F] [--pure-api-repeat 10] [--build]``.
"""
from __future__ import annotations

import argparse
import os
import re
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CLI = PKG / "wtc-compiler"


class RegressionFailed(Exception):
    pass


class Summary:
    def __init__(self, path: Path):
        self.path = path
        path.write_text("check\tstatus\tdetail\n")

    def _add(self, check, status, detail):
        line = f"{check}\t{status}\t{detail}"
        with open(self.path, "a") as f:
            f.write(line + "\n")
        print(line, file=sys.stdout if status == "PASS" else sys.stderr, flush=True)

    def ok(self, check, detail):
        self._add(check, "PASS", detail)

    def fail(self, check, detail):
        self._add(check, "FAIL", detail)
        raise RegressionFailed(f"{check}: {detail}")

    def require_file(self, check, path: Path):
        if not path.is_file():
            self.fail(check, f"missing file: {path}")
        self.ok(check, f"exists: {path}")

    def require_contains(self, check, path: Path, pattern: str):
        if not path.is_file() or not re.search(pattern, path.read_text()):
            self.fail(check, f"pattern '{pattern}' not found in {path}")
        self.ok(check, f"found '{pattern}' in {path}")


def default_inputs(out_base: Path) -> tuple[Path, Path]:
    from .chain_mlir import chain_mlir
    from .configs import ChainConfig
    cfg = ChainConfig("regression", 1, 8192, 128, 64, "f16", "f32", "uniform", 1.0)
    d = out_base / "inputs"
    d.mkdir(parents=True, exist_ok=True)
    plain, named = d / "matmul_softmax_chain_f16_native.mlir", d / "matmul_softmax_chain_named_softmax.mlir"
    plain.write_text(chain_mlir(cfg))
    named.write_text(chain_mlir(cfg, named_softmax=True))
    return plain, named


def run_regression(out_base: Path, input_mlir: Path | None = None,
                   named_input: Path | None = None, max_connect_level: int = 1,
                   pure_api_repeat: int = 10, build: bool = False, cli: Path = CLI) -> int:
    out_base.mkdir(parents=True, exist_ok=True)
    s = Summary(out_base / "regression_summary.tsv")
    try:
        if input_mlir is None or named_input is None:
            gen_plain, gen_named = default_inputs(out_base)
            input_mlir = input_mlir or gen_plain
            named_input = named_input or gen_named
        for p in (input_mlir, named_input):
            if not Path(p).is_file():
                print(f"error: input mlir not found: {p}", file=sys.stderr)
                return 2
        if build or not cli.exists():
            from . import build as B
            B.build()
        if not os.access(cli, os.X_OK):
            s.fail("build", f"wtc-compiler not found: {cli}")
        s.ok("build", str(cli))

        def wtc(check, *args):
            r = subprocess.run([str(cli), *map(str, args), "--max-connect-level",
                                str(max_connect_level)], capture_output=True, text=True, timeout=600)
            if r.returncode != 0:
                s.fail(check, f"wtc-compiler exited {r.returncode}: {r.stderr.strip()[-400:]}")

        d = out_base / "search_api"
        wtc("search_api", "--input", input_mlir, "--output-dir", d, "--backend-mode", "api",
            "--search-only")
        s.require_file("search_api.best", d / "search" / "best.json")
        s.require_file("search_api.candidates", d / "search" / "candidates.tsv")

        d = out_base / "search_named_softmax"
        wtc("named_softmax", "--input", named_input, "--output-dir", d, "--backend-mode",
            "process_chain", "--search-only")
        canon = d / "ir" / "01.canonicalized.mlir"
        s.require_file("named_softmax.canonicalized", canon)
        s.require_contains("named_softmax.exp", canon, r"math\.exp")
        s.require_contains("named_softmax.div", canon, r"arith\.divf")
        if re.search(r"linalg\.softmax", canon.read_text()):
            s.fail("named_softmax.decompose", "linalg.softmax remains after canonicalize")
        s.ok("named_softmax.decompose", "linalg.softmax removed after canonicalize")

        d = out_base / "full_api_default"
        wtc("full_api_default", "--input", input_mlir, "--output-dir", d, "--backend-mode", "api",
            "--fused")
        s.require_file("full_api_default.runnable", d / "fused" / "05.out.nvvm.runnable.mlir")
        s.require_contains("full_api_default.workgroup", d / "fused" / "04.after_workgroup_launch.mlir",
                           r"workgroup\(")
        s.require_contains("full_api_default.launchfunc", d / "fused" / "05.out.nvvm.runnable.mlir",
                           r"gpu\.launch_func")

        d = out_base / "pure_api_repeat"
        wtc("pure_api_repeat", "--input", input_mlir, "--output-dir", d, "--backend-mode", "api",
            "--pure-api-full", "--fused", "--repeat", pure_api_repeat)
        last = d / f"iter_{pure_api_repeat - 1}" / "fused" / "05.out.nvvm.runnable.mlir"
        s.require_file("pure_api_repeat.runnable", last)
        s.require_contains("pure_api_repeat.launchfunc", last, r"gpu\.launch_func")
    except RegressionFailed:
        return 1
    print("[wtc] regression passed")
    print(f"  summary: {s.path}")
    return 0


def main(argv=None) -> int:
    env = os.environ
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out-base", default=env.get("OUT_BASE", "/tmp/wtc_regression"))
    ap.add_argument("--input", default=env.get("INPUT_MLIR"))
    ap.add_argument("--named-softmax-input", default=env.get("NAMED_SOFTMAX_INPUT_MLIR"))
    ap.add_argument("--max-connect-level", type=int, default=int(env.get("MAX_CONNECT_LEVEL", "1")))
    ap.add_argument("--pure-api-repeat", type=int, default=int(env.get("PURE_API_REPEAT", "10")))
    ap.add_argument("--build", action="store_true", help="rebuild the native parts first")
    a = ap.parse_args(argv)
    if a.pure_api_repeat < 1:
        ap.error("--pure-api-repeat must be >= 1")
    return run_regression(Path(a.out_base), Path(a.input) if a.input else None,
                          Path(a.named_softmax_input) if a.named_softmax_input else None,
                          a.max_connect_level, a.pure_api_repeat, a.build)


if __name__ == "__main__":
    sys.exit(main())
