"""Pin a fused-vs-unfused A/B run as the performance guard's baseline.

The counterpart of the reference's bench/pin_baseline.sh:1-67: run the A/B
harness without verification into ``--run-out-base``, then copy its
``ab_summary.tsv``, ``ab_summary.csv``, ``speedup.tsv`` and
``search/best.json`` and, per variant (``baseline``, ``fused``), the compile's
stage files under the names the reference pins (03 / 04 / 04c / 05 MLIR,
pin_baseline.sh:44-51) and this build's own (canonical chain, kernel plan,
launch manifest, kernel report) into ``--baseline-dir``, and write ``manifest.txt`` (timestamp,
input, mode, connect level, run directory; this build adds the device and
the timing settings).

The run takes every option of ``run_ab`` (shape, dtypes, pattern, warmup,
iterations); ``--verify`` is ignored, as the reference pins with VERIFY=0.

Usage: ``python -m welder_typical_chain_amd.pin_baseline [--baseline-dir D]
[--run-out-base D] [run_ab options]``.
"""
from __future__ import annotations

import argparse
import datetime
import os
import shutil
import sys
from pathlib import Path

from . import run_ab
from .perf_guard import DEFAULT_BASELINE_DIR

# the reference's stage files (bench/pin_baseline.sh:44-51), then this build's own
STAGE_FILES = ("03.after_postbufferize.mlir", "04.after_workgroup_launch.mlir",
               "04c.after_linalg_to_loops.mlir", "05.out.nvvm.runnable.mlir")
VARIANT_FILES = STAGE_FILES + ("03.chain.canonical.mlir", "04.kernel.plan.json", "05.out.hip.launch.json",
                               "kernel_report.txt")
TOP_FILES = ("ab_summary.tsv", "ab_summary.csv", "speedup.tsv")


def pin(run_args, baseline_dir: Path) -> dict:
    run_args.verify = False
    run_base = Path(run_args.out_base)
    print("[wtc] run AB to pin baseline", flush=True)
    res = run_ab.run_ab(run_args)
    print(f"[wtc] pin artifacts to {baseline_dir}", flush=True)
    for sub in ("baseline", "fused", "search"):
        (baseline_dir / sub).mkdir(parents=True, exist_ok=True)
    for name in TOP_FILES:
        shutil.copyfile(run_base / name, baseline_dir / name)
    shutil.copyfile(run_base / "search" / "best.json", baseline_dir / "search" / "best.json")
    for variant in ("baseline", "fused"):
        for name in VARIANT_FILES:
            shutil.copyfile(run_base / variant / name, baseline_dir / variant / name)
    import torch
    device = "none"
    if torch.cuda.is_available():
        props = torch.cuda.get_device_properties(0)
        device = f"{props.name} ({props.gcnArchName}, {props.multi_processor_count} CUs)"
    input_mlir = run_args.input_mlir or str(run_base / "input.mlir")
    manifest = [
        f"timestamp={datetime.datetime.now().astimezone().isoformat(timespec='seconds')}",
        f"input_mlir={input_mlir}",
        "backend_mode=api",
        f"max_connect_level={run_args.max_connect_level}",
        f"run_out_base={run_base}",
        f"device={device}",
        f"pattern={run_args.pattern}",
        f"seed={run_args.seed}",
        f"warmup={run_args.warmup}",
        f"iters={run_args.iters}",
    ]
    (baseline_dir / "manifest.txt").write_text("\n".join(manifest) + "\n")
    print("[wtc] baseline pinned")
    print(f"  baseline_dir: {baseline_dir}")
    print(f"  manifest:     {baseline_dir / 'manifest.txt'}")
    return res


def main(argv=None) -> int:
    env = os.environ
    ap = argparse.ArgumentParser(add_help=False)
    ap.add_argument("--baseline-dir", default=env.get("BASELINE_DIR", str(DEFAULT_BASELINE_DIR)))
    ap.add_argument("--run-out-base", default=env.get("RUN_OUT_BASE", "/tmp/wtc_pin_baseline_run"))
    ours, rest = ap.parse_known_args(argv)
    run_args = run_ab.parse_args(rest + ["--out-base", ours.run_out_base])
    if run_args.input_mlir is None and env.get("INPUT_MLIR"):
        run_args.input_mlir = env["INPUT_MLIR"]
    pin(run_args, Path(ours.baseline_dir))
    return 0


if __name__ == "__main__":
    sys.exit(main())
