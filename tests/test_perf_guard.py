"""The performance guard, the baseline pin and the artefact regression run
(counterparts of the reference's bench/check_perf_guard.sh,
bench/pin_baseline.sh and bench/run_regression.sh).

CPU: every guard mode and error status on hand-written A/B summaries, the
pinned baseline shipped with the package, and the regression run over the
wtc-compiler CLI.  GPU: a pin of a real A/B run, guarded against itself
and against a slowed copy.
"""
from __future__ import annotations

import shutil
from pathlib import Path

import pytest

from welder_typical_chain_amd import perf_guard as PG
from welder_typical_chain_amd import regression as RG

HEADER = "case\tavg_ms\tkernels\tpattern\tseed\titers\twarmup\tout_dir\n"


def write_ab(d: Path, baseline_ms, fused_ms, speedup=None):
    d.mkdir(parents=True, exist_ok=True)
    (d / "ab_summary.tsv").write_text(
        HEADER + f"baseline\t{baseline_ms}\t5\tlinear\t1\t200\t10\t{d}/baseline\n"
        f"fused\t{fused_ms}\t1\tlinear\t1\t200\t10\t{d}/fused\n")
    sp = baseline_ms / fused_ms if speedup is None else speedup
    (d / "speedup.tsv").write_text(f"speedup\t{sp:.4f}\n")
    return d


def run_guard(base, cur, pct=3.0, mode="auto"):
    import io
    out, err = io.StringIO(), io.StringIO()
    rc = PG.guard(base, cur, pct, mode, out=out, err=err)
    return rc, out.getvalue(), err.getvalue()


def test_identical_runs_pass(tmp_path):
    base = write_ab(tmp_path / "base", 0.025, 0.006)
    rc, out, _ = run_guard(base, base)
    assert rc == 0
    assert "PASS baseline.avg_ms" in out and "PASS fused.avg_ms" in out and "PASS speedup" in out
    assert "[wtc] perf guard passed" in out


def test_threshold_is_inclusive_and_relative(tmp_path):
    base = write_ab(tmp_path / "base", 1.0, 0.5)
    # exactly 3 % slower fused, same baseline: the fused time passes at its
    # limit, the speedup (2 / 1.03 = 1.9417 against a floor of 1.94) too
    at = write_ab(tmp_path / "at", 1.0, 0.515)
    assert run_guard(base, at)[0] == 0
    over = write_ab(tmp_path / "over", 1.0, 0.5155)
    rc, _, err = run_guard(base, over)
    assert rc == 1 and "FAIL fused.avg_ms" in err and "limit=0.515" in err
    # a larger threshold lets it through
    assert run_guard(base, over, pct=5.0)[0] == 0


def test_baseline_regression_fails_first(tmp_path):
    base = write_ab(tmp_path / "base", 1.0, 0.5)
    cur = write_ab(tmp_path / "cur", 1.2, 0.5)
    rc, out, err = run_guard(base, cur)
    assert rc == 1 and "FAIL baseline.avg_ms" in err and "fused.avg_ms" not in out + err


def test_speedup_modes(tmp_path):
    base = write_ab(tmp_path / "base", 1.0, 0.5)                    # speedup 2.0
    # the baseline got 10 % faster, fused unchanged: speedup 1.8 (-10 %)
    faster_base = write_ab(tmp_path / "fb", 0.9, 0.5)
    rc, out, _ = run_guard(base, faster_base, mode="auto")
    assert rc == 0 and "SKIP speedup: baseline improved beyond 3%" in out
    rc, _, err = run_guard(base, faster_base, mode="strict")
    assert rc == 1 and "FAIL speedup" in err and "min_allowed=1.94" in err
    rc, out, _ = run_guard(base, faster_base, mode="off")
    assert rc == 0 and "SKIP speedup: SPEEDUP_CHECK_MODE=off" in out
    # a speedup file that disagrees with the times is taken as written: with
    # the baseline within threshold, auto checks it
    low = write_ab(tmp_path / "low", 1.0, 0.5, speedup=1.5)
    rc, _, err = run_guard(base, low, mode="auto")
    assert rc == 1 and "FAIL speedup" in err
    assert run_guard(base, low, mode="off")[0] == 0


def test_missing_files_invalid_mode_and_bad_values(tmp_path):
    base = write_ab(tmp_path / "base", 1.0, 0.5)
    rc, _, err = run_guard(base, tmp_path / "nowhere")
    assert rc == 2 and "missing required file" in err
    rc, _, err = run_guard(base, base, mode="loose")
    assert rc == 2 and "invalid SPEEDUP_CHECK_MODE=loose" in err
    bad = write_ab(tmp_path / "bad", 1.0, 0.5)
    (bad / "ab_summary.tsv").write_text(HEADER + "baseline\t1.0\t5\n")   # no fused row
    assert run_guard(base, bad)[0] == 2
    (bad / "ab_summary.tsv").write_text(HEADER + "baseline\tx\t5\nfused\t0.5\t1\n")
    assert run_guard(base, bad)[0] == 2
    write_ab(bad, 1.0, 0.5)
    (bad / "speedup.tsv").write_text("speedup\tnan\n")       # run_ab writes nan for a 0 ms fused time
    assert run_guard(base, bad)[0] == 2
    (bad / "speedup.tsv").write_text("")
    assert run_guard(base, bad)[0] == 2


def test_environment_sets_the_defaults(tmp_path, monkeypatch):
    base = write_ab(tmp_path / "base", 1.0, 0.5)
    cur = write_ab(tmp_path / "cur", 1.0, 0.52)                # +4 %
    monkeypatch.setenv("BASELINE_DIR", str(base))
    monkeypatch.setenv("CURRENT_OUT_BASE", str(cur))
    assert PG.main([]) == 1
    monkeypatch.setenv("MAX_REGRESSION_PCT", "5")
    assert PG.main([]) == 0
    monkeypatch.setenv("SPEEDUP_CHECK_MODE", "bogus")
    assert PG.main([]) == 2
    assert PG.main(["--speedup-check-mode", "off", "--max-regression-pct", "x"]) == 2


def test_shipped_baseline_is_complete():
    """The pinned MI355X A/B run shipped with the package parses and guards
    itself."""
    d = PG.DEFAULT_BASELINE_DIR
    if not (d / "ab_summary.tsv").exists():
        pytest.skip("no pinned baseline shipped")
    assert run_guard(d, d)[0] == 0
    for name in ("ab_summary.csv", "manifest.txt", "search/best.json"):
        assert (d / name).is_file(), name
    for variant in ("baseline", "fused"):
        for name in ("03.after_postbufferize.mlir", "04.after_workgroup_launch.mlir",
                     "04c.after_linalg_to_loops.mlir", "05.out.nvvm.runnable.mlir",
                     "03.chain.canonical.mlir", "04.kernel.plan.json", "05.out.hip.launch.json",
                     "kernel_report.txt"):
            assert (d / variant / name).is_file(), (variant, name)
    assert PG.read_avg_ms(d / "ab_summary.tsv", "fused") < PG.read_avg_ms(d / "ab_summary.tsv", "baseline")


def test_regression_run_passes(native_lib, tmp_path):
    rc = RG.run_regression(tmp_path / "reg", pure_api_repeat=3)
    assert rc == 0
    rows = (tmp_path / "reg" / "regression_summary.tsv").read_text().splitlines()
    assert rows[0] == "check\tstatus\tdetail"
    checks = [r.split("\t") for r in rows[1:]]
    assert all(status == "PASS" for _, status, _ in checks)
    assert [c for c, _, _ in checks] == [
        "build", "search_api.best", "search_api.candidates", "named_softmax.canonicalized",
        "named_softmax.exp", "named_softmax.div", "named_softmax.decompose",
        "full_api_default.runnable", "full_api_default.workgroup", "full_api_default.launchfunc",
        "pure_api_repeat.runnable", "pure_api_repeat.launchfunc"]
    assert (tmp_path / "reg" / "pure_api_repeat" / "iter_2" / "fused").is_dir()


def test_regression_stops_at_the_first_failure(native_lib, tmp_path):
    plain, _ = RG.default_inputs(tmp_path / "gen")
    not_a_chain = tmp_path / "bad.mlir"
    not_a_chain.write_text("func.func @f() { return }\n")
    rc = RG.run_regression(tmp_path / "reg", input_mlir=plain, named_input=not_a_chain)
    assert rc == 1
    rows = (tmp_path / "reg" / "regression_summary.tsv").read_text().splitlines()
    assert rows[-1].startswith("named_softmax\tFAIL\twtc-compiler exited 1")
    assert not (tmp_path / "reg" / "full_api_default").exists()
    assert RG.run_regression(tmp_path / "r2", input_mlir=tmp_path / "missing.mlir",
                             named_input=plain) == 2


@pytest.mark.gpu
def test_pin_then_guard_on_gpu(native_lib, tmp_path):
    from welder_typical_chain_amd import pin_baseline as PB
    from welder_typical_chain_amd import run_ab as AB
    print("case: pin_baseline m=2048 n=128 k=64 f16->f32, iters 50", flush=True)
    pinned = tmp_path / "pinned"
    run_dir = tmp_path / "run"
    args = AB.parse_args(["--out-base", str(run_dir), "--m", "2048", "--iters", "50", "--verify"])
    res = PB.pin(args, pinned)
    assert args.verify is False and res["verify"] == {}
    for name in ("ab_summary.tsv", "ab_summary.csv", "speedup.tsv", "manifest.txt",
                 "search/best.json", "fused/05.out.hip.launch.json", "baseline/04.kernel.plan.json",
                 "fused/04c.after_linalg_to_loops.mlir", "baseline/05.out.nvvm.runnable.mlir"):
        assert (pinned / name).is_file(), name
    manifest = dict(l.split("=", 1) for l in (pinned / "manifest.txt").read_text().splitlines())
    assert manifest["run_out_base"] == str(run_dir) and manifest["iters"] == "50"
    assert run_guard(pinned, run_dir)[0] == 0          # the run the pin came from
    slowed = tmp_path / "slowed"
    shutil.copytree(run_dir, slowed, ignore=shutil.ignore_patterns("baseline", "fused", "search"))
    ms_b = PG.read_avg_ms(run_dir / "ab_summary.tsv", "baseline")
    ms_f = PG.read_avg_ms(run_dir / "ab_summary.tsv", "fused")
    write_ab(slowed, ms_b, ms_f * 1.5)
    rc, _, err = run_guard(pinned, slowed)
    assert rc == 1 and "FAIL fused.avg_ms" in err
