"""Performance guard: the current fused-vs-unfused A/B run against a pinned one.

The counterpart of the reference's bench/check_perf_guard.sh:1-121.  Both
directories hold what ``run_ab`` writes (``ab_summary.tsv`` and
``speedup.tsv``); the pinned one is made by ``pin_baseline``.  Checks:

- ``baseline.avg_ms`` and ``fused.avg_ms`` may be at most ``max_regression_pct``
  percent slower than the pinned values (check_perf_guard.sh:60-75,104-105);
- the speedup may be at most that many percent lower, depending on the mode
  (check_perf_guard.sh:9-14,107-121):
  ``strict`` always checks it, ``off`` never does, and ``auto`` (the
  default) skips it when the current unfused baseline is more than the
  threshold faster than the pinned one, since a faster baseline shrinks the
  speedup without the fused kernel getting any slower.

Exit status: 0 pass, 1 a check failed, 2 a file is missing, a value does not
parse or the mode is unknown (check_perf_guard.sh:22-27,52-57,118-120).

The reference's environment variables (BASELINE_DIR, CURRENT_OUT_BASE,
MAX_REGRESSION_PCT, SPEEDUP_CHECK_MODE) set the defaults of the flags.

Usage: ``python -m welder_typical_chain_amd.perf_guard [--baseline-dir D]
[--current-out D] [--max-regression-pct 3] [--speedup-check-mode auto]``.
"""
from __future__ import annotations

import argparse
import math
import os
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
DEFAULT_BASELINE_DIR = PKG / "baselines" / "default"
MODES = ("auto", "strict", "off")


class GuardError(Exception):
    """A missing file or an unparseable value (exit status 2)."""


def _number(text: str, what: str) -> float:
    try:
        v = float(text)
    except ValueError:
        raise GuardError(f"failed to parse performance metrics ({what}: {text!r})") from None
    if math.isnan(v):
        raise GuardError(f"failed to parse performance metrics ({what} is nan)")
    return v


def read_avg_ms(path: Path, case: str) -> float:
    """avg_ms (second column) of the first row whose first column is `case`."""
    for line in path.read_text().splitlines():
        cols = line.split("\t")
        if cols[0] == case and len(cols) > 1:
            return _number(cols[1], f"{path}:{case}")
    raise GuardError(f"failed to parse performance metrics (no '{case}' row in {path})")


def read_speedup(path: Path) -> float:
    """Second field of the first line of speedup.tsv."""
    lines = path.read_text().splitlines()
    cols = lines[0].split("\t") if lines else []
    if len(cols) < 2:
        raise GuardError(f"failed to parse performance metrics ({path})")
    return _number(cols[1], str(path))


def not_worse_than(name: str, base: float, cur: float, pct: float) -> tuple[bool, str]:
    """Time-like metric: current <= pinned * (1 + pct/100)."""
    limit = base * (1.0 + pct / 100.0)
    if cur <= limit:
        return True, f"PASS {name}: baseline={base:.9g}, current={cur:.9g}, threshold={pct:g}%"
    return False, (f"FAIL {name}: baseline={base:.9g}, current={cur:.9g}, limit={limit:.9g} "
                   f"({pct:g}% regression threshold)")


def not_less_than(name: str, base: float, cur: float, pct: float) -> tuple[bool, str]:
    """Higher-is-better metric: current >= pinned * (1 - pct/100)."""
    limit = base * (1.0 - pct / 100.0)
    if cur >= limit:
        return True, f"PASS {name}: baseline={base:.9g}, current={cur:.9g}, drop_threshold={pct:g}%"
    return False, (f"FAIL {name}: baseline={base:.9g}, current={cur:.9g}, min_allowed={limit:.9g} "
                   f"({pct:g}% drop threshold)")


def guard(baseline_dir: Path, current_out: Path, max_regression_pct: float = 3.0,
          speedup_check_mode: str = "auto", out=sys.stdout, err=sys.stderr) -> int:
    baseline_dir, current_out = Path(baseline_dir), Path(current_out)
    files = {"base_ab": baseline_dir / "ab_summary.tsv", "base_sp": baseline_dir / "speedup.tsv",
             "cur_ab": current_out / "ab_summary.tsv", "cur_sp": current_out / "speedup.tsv"}
    for p in files.values():
        if not p.is_file():
            print(f"error: missing required file: {p}", file=err)
            return 2
    if speedup_check_mode not in MODES:
        print(f"error: invalid SPEEDUP_CHECK_MODE={speedup_check_mode} (expected auto|strict|off)",
              file=err)
        return 2
    try:
        base_b = read_avg_ms(files["base_ab"], "baseline")
        base_f = read_avg_ms(files["base_ab"], "fused")
        cur_b = read_avg_ms(files["cur_ab"], "baseline")
        cur_f = read_avg_ms(files["cur_ab"], "fused")
        base_s = read_speedup(files["base_sp"])
        cur_s = read_speedup(files["cur_sp"])
    except GuardError as e:
        print(f"error: {e}", file=err)
        return 2

    def report(res):
        ok, msg = res
        print(msg, file=out if ok else err)
        return ok

    pct = max_regression_pct
    if not report(not_worse_than("baseline.avg_ms", base_b, cur_b, pct)):
        return 1
    if not report(not_worse_than("fused.avg_ms", base_f, cur_f, pct)):
        return 1
    check_speedup = speedup_check_mode == "strict"
    if speedup_check_mode == "off":
        print("SKIP speedup: SPEEDUP_CHECK_MODE=off", file=out)
    elif speedup_check_mode == "auto":
        if cur_b < base_b * (1.0 - pct / 100.0):
            print(f"SKIP speedup: baseline improved beyond {pct:g}% "
                  f"(baseline={base_b:.9g}, current={cur_b:.9g})", file=out)
        else:
            check_speedup = True
    if check_speedup and not report(not_less_than("speedup", base_s, cur_s, pct)):
        return 1
    print("[wtc] perf guard passed", file=out)
    print(f"  baseline_dir: {baseline_dir}", file=out)
    print(f"  current_out:  {current_out}", file=out)
    return 0


def parse_args(argv=None):
    env = os.environ
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--baseline-dir", default=env.get("BASELINE_DIR", str(DEFAULT_BASELINE_DIR)))
    ap.add_argument("--current-out", default=env.get("CURRENT_OUT_BASE", "/tmp/wtc_ab"))
    ap.add_argument("--max-regression-pct", default=env.get("MAX_REGRESSION_PCT", "3"))
    ap.add_argument("--speedup-check-mode", default=env.get("SPEEDUP_CHECK_MODE", "auto"))
    return ap.parse_args(argv)


def main(argv=None) -> int:
    args = parse_args(argv)
    try:
        pct = float(args.max_regression_pct)
    except ValueError:
        print(f"error: invalid MAX_REGRESSION_PCT={args.max_regression_pct}", file=sys.stderr)
        return 2
    return guard(Path(args.baseline_dir), Path(args.current_out), pct, args.speedup_check_mode)


if __name__ == "__main__":
    sys.exit(main())
