"""CPU tests of the variant cost model (csrc/variants.cpp) against the
MI355X timing table it was fitted to (welder_typical_chain_amd/
calibration_mi355x.jsonl: every variant on every path it runs, back-to-back
calls, 60 shapes in four sets).

* AUTO's pick, priced at its measured time, is close to the measured
  fastest choice on every shape, and close on average;
* the constants in the C++ source are the fit of that table
  (calibrate.fit_constants reproduces its estimates);
* fitted on three sets and scored on the fourth, in turn, the ranking
  stays close (the model generalises to shapes it was not fitted to).
"""
from __future__ import annotations

import json
from pathlib import Path

import pytest

from welder_typical_chain_amd import _lib, calibrate

TABLE = Path(calibrate.__file__).resolve().parent / "calibration_mi355x.jsonl"
CODES = {"f32": 0, "f16": 1, "bf16": 2, "fp8": 3}
PATHS = {"exchange": 1, "split": 2, "unfused": 3, "rows": 4}


@pytest.fixture(scope="module")
def records(native_lib):
    return [json.loads(line) for line in TABLE.read_text().splitlines() if line.strip()]


def _by_shape(records):
    by = {}
    for r in records:
        if r["path"] != "unfused":
            by.setdefault(r["shape"], []).append(r)
    return by


def test_table_covers_every_variant_and_path(records):
    seen = {(r["in"], tuple(r["tiles"]), r["path"]) for r in records}
    for in_dt, code in CODES.items():
        for name, tiles, mask in _lib.variants(code):
            for path, p in PATHS.items():
                if mask & (1 << p):
                    assert (in_dt, tuple(tiles), path) in seen, (in_dt, name, path)
    assert len(_by_shape(records)) == 60


def test_auto_pick_is_close_to_the_measured_fastest(records):
    losses = {}
    for shape, rs in _by_shape(records).items():
        r0 = rs[0]
        pl = _lib.plan(r0["batch"], r0["m"], r0["n"], r0["k"], CODES[r0["in"]], CODES[r0["out"]],
                       _lib.PATH_AUTO, None, 256, 1)
        pick = [r for r in rs if r["tiles"] == pl["tiles"] and PATHS[r["path"]] == pl["path"]]
        assert len(pick) == 1, shape
        losses[shape] = pick[0]["us"] / min(r["us"] for r in rs) - 1
    mean = sum(losses.values()) / len(losses)
    worst = max(losses, key=losses.get)
    print(f"mean loss {100 * mean:.2f} %, worst {worst} {100 * losses[worst]:.1f} %")
    assert mean < 0.015
    assert losses[worst] < 0.15
    # the headline configurations
    for shape in ("c1_f32", "c2", "c3", "c4"):
        assert losses[shape] == 0.0, shape
    assert losses["c5"] < 0.015


def test_source_constants_are_the_fit_of_the_table(records):
    x = calibrate.fit_constants(records)
    worst = 0.0
    for r in records:
        if r["path"] == "unfused":
            continue
        cpp = _lib.plan(r["batch"], r["m"], r["n"], r["k"], CODES[r["in"]], CODES[r["out"]],
                        PATHS[r["path"]], r["tiles"], 256, 1)["est_us"]
        worst = max(worst, abs(calibrate.model_us(x, r) / cpp - 1))
    assert worst < 0.01, f"C++ estimates differ from the table's fit by up to {100 * worst:.2f} %"


def test_ranking_generalises_to_held_out_sets(records):
    losses = []
    for held in ("fit", "validation", "holdout", "extra"):
        x = calibrate.fit_constants([r for r in records if r["set"] != held])
        losses += list(calibrate.ranking_losses(x, [r for r in records if r["set"] == held]).values())
    assert sum(losses) / len(losses) < 0.02
    assert max(losses) < 0.2
