"""The fused-vs-unfused A/B harness (welder_typical_chain_amd.run_ab).

CPU: the input patterns against the oracle's generators (bit-exact), the
dump descriptor round trip, the verifier's pass rule against the oracle's
float64 rows, and the solve + compile pair.  GPU: the whole harness on small
chains, including its own verification of both cases.
"""
from __future__ import annotations

import csv
import json
import re

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from welder_typical_chain_amd import run_ab as AB  # noqa: E402


def _xorshift_loop(n, seed):
    s = seed or 1
    out = []
    for _ in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out.append(s)
    return np.array(out, dtype=np.uint32)


@pytest.mark.parametrize("n", [0, 1, 2, 3, 31, 64, 1000, 4097])
@pytest.mark.parametrize("seed", [0, 1, 12345, 0xFFFFFFFF])
def test_xorshift_doubling_matches_the_sequential_stream(n, seed):
    np.testing.assert_array_equal(AB.xorshift32_states(n, seed), _xorshift_loop(n, seed))


@pytest.mark.parametrize("seed", [0, 1, 7])
def test_random_pattern_matches_oracle(seed):
    np.testing.assert_array_equal(AB.pattern_values("random", 70001, seed), O.fill_random(70001, seed))


def test_linear_and_zero_patterns_match_oracle():
    np.testing.assert_array_equal(AB.pattern_values("linear", 5000, 3), O.fill_linear(5000))
    assert not AB.pattern_values("zero", 100, 1).any()
    with pytest.raises(ValueError):
        AB.pattern_values("gauss", 4, 1)


@pytest.mark.parametrize("dtype,shape", [("f32", (5, 7)), ("f16", (3, 4, 6)), ("bf16", (8, 16))])
def test_dump_round_trip(tmp_path, dtype, shape):
    vals = np.random.default_rng(0).random(shape).astype(np.float32)
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dtype]
    t = torch.from_numpy(vals).to(tdt)
    raw = t.view(torch.int16 if t.element_size() == 2 else torch.int32).numpy().tobytes()
    AB.write_dump(tmp_path / "out.bin", raw, shape, dtype)
    meta = json.loads((tmp_path / "out.bin.json").read_text())
    assert meta["rank"] == len(shape) and meta["sizes"] == list(shape)
    assert meta["elem_bytes"] == t.element_size() and meta["bytes"] == len(raw)
    assert meta["strides"][-1] == 1 and meta["offset"] == 0
    got, _ = AB.read_dump(tmp_path / "out.bin")
    np.testing.assert_array_equal(got, t.float().numpy().astype(np.float64))


def _exact_dump(tmp_path, m, n, k, pattern, seed, scale=1.0):
    a = AB.pattern_values(pattern, m * k, seed).reshape(m, k)
    b = AB.pattern_values(pattern, k * n, seed).reshape(k, n)
    _, probs = O.chain_rows(a, b, list(range(m)), scale)
    out = probs.astype(np.float32)
    AB.write_dump(tmp_path / "out.bin", out.tobytes(), (m, n), "f32")
    return out


@pytest.mark.parametrize("pattern", ["linear", "random"])
def test_verifier_pass_rule(tmp_path, pattern):
    m, n, k = 40, 24, 16
    out = _exact_dump(tmp_path, m, n, k, pattern, 3, scale=0.5)
    ok, msg = AB.verify_dump(tmp_path / "out.bin", k=k, pattern=pattern, seed=3, in_dtype="f32",
                             rtol=1e-3, atol=1e-3, logit_scale=0.5)
    assert ok and msg.startswith("PASS") and "rows=7" in msg, msg   # rows 0,1,2,3,7,15,31 < 40
    # a wrong scale, a perturbed sampled entry, and a NaN each fail
    assert not AB.verify_dump(tmp_path / "out.bin", k=k, pattern=pattern, seed=3, in_dtype="f32",
                              rtol=1e-3, atol=1e-3, logit_scale=1.0)[0]
    bad = out.copy()
    bad[15, 5] += 3e-3
    AB.write_dump(tmp_path / "out.bin", bad.tobytes(), (m, n), "f32")
    assert not AB.verify_dump(tmp_path / "out.bin", k=k, pattern=pattern, seed=3, in_dtype="f32",
                              rtol=1e-3, atol=1e-3, logit_scale=0.5)[0]
    bad = out.copy()
    bad[16, 5] += 0.5   # row 16 is not sampled
    AB.write_dump(tmp_path / "out.bin", bad.tobytes(), (m, n), "f32")
    assert AB.verify_dump(tmp_path / "out.bin", k=k, pattern=pattern, seed=3, in_dtype="f32",
                          rtol=1e-3, atol=1e-3, logit_scale=0.5)[0]
    bad = out.copy()
    bad[0, 0] = np.nan
    AB.write_dump(tmp_path / "out.bin", bad.tobytes(), (m, n), "f32")
    ok, msg = AB.verify_dump(tmp_path / "out.bin", k=k, pattern=pattern, seed=3, in_dtype="f32",
                             rtol=1e-3, atol=1e-3, logit_scale=0.5)
    assert not ok and "NaN" in msg


def test_solve_and_compile_pair(native_lib, tmp_path):
    args = AB.parse_args(["--out-base", str(tmp_path), "--m", "512", "--n", "256", "--k", "64"])
    src = AB._default_chain(args)
    tiles = AB.solve_tiles(native_lib, src, tmp_path / "search")
    best = (tmp_path / "search" / "best.json").read_text()
    # read the way the reference reads it: first match of "key"\s*:\s*(-?[0-9]+)
    parsed = [int(re.search(rf'"{kk}"\s*:\s*(-?[0-9]+)', best).group(1))
              for kk in ("tileM", "tileN", "tileK", "threadTileM", "threadTileN")]
    assert parsed == tiles
    base = AB.compile_case(native_lib, src, tmp_path / "baseline", tiles, fused=False)
    fused = AB.compile_case(native_lib, src, tmp_path / "fused", tiles, fused=True)
    assert base["path"] == "unfused" and fused["path"] != "unfused"
    assert AB.kernel_count(tmp_path / "baseline") == 5
    assert AB.kernel_count(tmp_path / "fused") in (1, 2)
    assert (base["problem"]["m"], base["problem"]["n"], base["problem"]["k"]) == (512, 256, 64)
    assert base["in_dtype"] == "f16" and base["out_dtype"] == "f32"


# ---- GPU: the whole harness --------------------------------------------------------

needs_gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="no GPU")


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("argv", [
    ["--m", "512", "--n", "256", "--k", "64"],
    ["--m", "256", "--n", "2048", "--k", "128", "--pattern", "random", "--seed", "7",
     "--in-dtype", "bf16", "--out-dtype", "f16"],
    ["--batch", "3", "--m", "256", "--n", "512", "--k", "64", "--logit-scale", "0.125",
     "--pattern", "random", "--out-dtype", "f16"],
], ids=["f16-f32-linear", "bf16-f16-random", "batched-f16-scaled"])
def test_ab_harness_end_to_end(native_lib, tmp_path, argv):
    print(f"\n[gpu-case] run_ab {' '.join(argv)}", flush=True)
    args = AB.parse_args(argv + ["--out-base", str(tmp_path), "--warmup", "2", "--iters", "5",
                                 "--verify"])
    res = AB.run_ab(args)
    assert res["verify"] == {"baseline": True, "fused": True}
    rows = list(csv.reader(open(tmp_path / "ab_summary.tsv"), delimiter="\t"))
    assert tuple(rows[0]) == AB.SUMMARY_HEADER
    assert [r[0] for r in rows[1:]] == ["baseline", "fused"]
    assert rows[1][2] == "5" and rows[2][2] in ("1", "2")
    for r in rows[1:]:
        assert float(r[1]) > 0 and r[3] == args.pattern and r[5] == "5" and r[6] == "2"
        assert (tmp_path / r[0] / "out.bin").exists() and (tmp_path / r[0] / "verify.log").exists()
    assert list(csv.reader(open(tmp_path / "ab_summary.csv")))[1:] == rows[1:]
    sp = (tmp_path / "speedup.tsv").read_text().split("\t")
    assert sp[0] == "speedup"
    # the summary's times are printed to 1 ns, so their ratio carries their
    # rounding: a relative check (a 5 us fused call already allows 1e-4)
    ratio = float(rows[1][1]) / float(rows[2][1])
    assert abs(float(sp[1]) - ratio) <= 1e-3 * ratio
    # the two cases computed the same chain
    ob, _ = AB.read_dump(tmp_path / "baseline" / "out.bin")
    of, _ = AB.read_dump(tmp_path / "fused" / "out.bin")
    np.testing.assert_allclose(ob, of, atol=2e-3, rtol=1e-2)
