"""CPU tests of the C-ABI library: exports, launch planning, argument errors,
and the compile / solver entry points on chain MLIR files.  Nothing here
launches a kernel (no GPU in this container)."""
from __future__ import annotations

import ctypes
import json
import re
from pathlib import Path

import pytest

from welder_typical_chain_amd import _lib
from welder_typical_chain_amd.chain_mlir import chain_mlir
from welder_typical_chain_amd.configs import CONFIGS, ChainConfig

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "welder_typical_chain_amd"
REF_MLIR = Path("/root/reference/mlir")


def declared_functions() -> set[str]:
    """Every function the public headers declare."""
    names = set()
    for h in (ROOT / "include" / "wtc").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b((?:wtc|welder)_\w+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def L(native_lib):
    return _lib.lib()


def test_every_declared_symbol_is_exported(L):
    names = declared_functions()
    assert {"wtc_matmul_softmax", "welder_compile_typical_chain_to_nvvm",
            "welder_solver_solve_typical_chain"} <= names
    for n in sorted(names):
        assert hasattr(L, n), f"{n} declared in include/wtc but not exported"
    assert names <= set(_lib.SIGNATURES), "ctypes prototypes missing for some declarations"


def test_reference_named_libraries():
    comp = ctypes.CDLL(str(PKG / "libwelder-compile-capi.so"))
    assert hasattr(comp, "welder_compile_typical_chain_to_nvvm")
    solver = ctypes.CDLL(str(PKG / "libwelder-solver-capi.so"))
    assert hasattr(solver, "welder_solver_solve_typical_chain")


def test_phase_stamps_only_in_the_profiling_build(L):
    """The stamp reader exists only in libwtc_hip_stamps.so, which exports the
    same C-ABI; the product library has no stamps."""
    assert not hasattr(L, "wtc_phase_stamps_read")
    S = _lib.stamps_lib()
    assert hasattr(S, "wtc_phase_stamps_read")
    for n in sorted(declared_functions()):
        assert hasattr(S, n), n


def test_version(L):
    assert b"gfx950" in L.wtc_version()


def plan(L, batch, m, n, k, i, o, path, cu=256, wg=1):
    grid, ws = ctypes.c_int64(), ctypes.c_int64()
    chosen = ctypes.c_int()
    rc = L.wtc_plan(batch, m, n, k, i, o, path, cu, wg, ctypes.byref(grid), ctypes.byref(chosen),
                    ctypes.byref(ws))
    return rc, grid.value, chosen.value, ws.value


def test_plan_headline_and_configs(L):
    # C2: 16 x 16 tiles, one per CU -> one-launch exchange path
    rc, grid, path, ws = plan(L, 1, 2048, 2048, 1024, _lib.DTYPE_F16, _lib.DTYPE_F16, _lib.PATH_AUTO)
    assert (rc, grid, path) == (0, 256, _lib.PATH_EXCHANGE)
    assert ws == L.wtc_matmul_softmax_workspace_size(1, 2048, 2048, 1024, 1, 1, 0)
    # diagnostic words, 1024 slot generation words, then 256 slots x 128 tagged
    # 8-byte entries (the split path's statistics need the same 2048 x 16 x 8)
    assert ws >= 256 + 1024 * 4 + 256 * 128 * 8
    # C3: k = 128 and 64 x 16 row blocks -> one workgroup per row block
    rc, grid, path, _ = plan(L, 64, 2048, 2048, 128, 1, 1, _lib.PATH_AUTO)
    assert (rc, grid, path) == (0, 64 * 16, _lib.PATH_ROWS)
    rc, grid, path, _ = plan(L, 64, 2048, 2048, 128, 1, 1, _lib.PATH_SPLIT)
    assert (rc, grid, path) == (0, 64 * 8 * 8, _lib.PATH_SPLIT)  # 256x256 tiles
    # the rows path needs 16-bit inputs and k <= 128
    assert plan(L, 64, 2048, 2048, 256, 1, 1, _lib.PATH_AUTO)[2] == _lib.PATH_SPLIT
    assert plan(L, 64, 2048, 2048, 128, _lib.DTYPE_FP8_E4M3, 1, _lib.PATH_AUTO)[2] == _lib.PATH_SPLIT
    rc, *_ = plan(L, 1, 256, 256, 256, 1, 1, _lib.PATH_ROWS)
    assert rc == _lib.WTC_ERR_UNSUPPORTED and b"rows path" in L.wtc_last_error()
    # C4: 256 column tiles per row -> split, with 256x256 tiles (4 x 128)
    rc, grid, path, _ = plan(L, 1, 1024, 32768, 4096, _lib.DTYPE_BF16, 1, _lib.PATH_AUTO)
    assert (rc, grid, path) == (0, 4 * 128, _lib.PATH_SPLIT)
    # C5 (fp8): split, 256x256 tiles (32 x 32)
    rc, grid, path, _ = plan(L, 1, 8192, 8192, 4096, _lib.DTYPE_FP8_E4M3, 1, _lib.PATH_AUTO)
    assert (rc, grid, path) == (0, 32 * 32, _lib.PATH_SPLIT)
    # f32 has one layout (128-row tiles)
    assert plan(L, 1, 1024, 32768, 64, _lib.DTYPE_F32, 0, _lib.PATH_SPLIT)[1] == 8 * 256
    # forcing the exchange path where it cannot be co-resident is refused
    rc, *_ = plan(L, 1, 1024, 32768, 4096, _lib.DTYPE_BF16, 1, _lib.PATH_EXCHANGE)
    assert rc == _lib.WTC_ERR_UNSUPPORTED and b"co-resident" in L.wtc_last_error()
    # ragged: 200 x 264 -> 2 x 3 tiles
    rc, grid, path, _ = plan(L, 1, 200, 264, 72, 1, 1, _lib.PATH_AUTO)
    assert (rc, grid, path) == (0, 6, _lib.PATH_EXCHANGE)
    # unfused needs room for the f32 logits
    _, _, _, ws_u = plan(L, 1, 2048, 2048, 1024, 1, 1, _lib.PATH_UNFUSED)
    assert ws_u >= ws + 2048 * 2048 * 4


F16, BF16, FP8, F32 = _lib.DTYPE_F16, _lib.DTYPE_BF16, _lib.DTYPE_FP8_E4M3, _lib.DTYPE_F32
T128 = {F16: [128, 128, 64, 2, 16], BF16: [128, 128, 64, 2, 16], FP8: [128, 128, 128, 2, 16]}
LDR = {F16: [128, 128, 64, 2, 32], BF16: [128, 128, 64, 2, 32], FP8: [128, 128, 128, 2, 32]}
T256 = {F16: [256, 128, 64, 2, 32], BF16: [256, 128, 64, 2, 32], FP8: [256, 128, 128, 2, 32]}
W256 = {F16: [256, 256, 32, 4, 64], BF16: [256, 256, 32, 4, 64], FP8: [256, 256, 64, 4, 64]}
ROWS = [128, 128, 128, 2, 16]


def test_variant_table(L):
    """Five variants for 16-bit inputs, four for fp8 (no rows kernel), one
    for f32, in id order; tiles distinct within an input type; each runs the
    paths its kernels implement."""
    ex, sp, un, ro = (1 << _lib.PATH_EXCHANGE, 1 << _lib.PATH_SPLIT, 1 << _lib.PATH_UNFUSED,
                      1 << _lib.PATH_ROWS)
    for dt in (F16, BF16):
        vs = _lib.variants(dt)
        assert [v[1] for v in vs] == [T128[dt], LDR[dt], T256[dt], ROWS, W256[dt]]
        assert [v[2] for v in vs] == [ex | sp | un, ex | sp | un, sp | un, ro, sp | un]
    assert [v[1] for v in _lib.variants(FP8)] == [T128[FP8], LDR[FP8], T256[FP8], W256[FP8]]
    assert [v[1] for v in _lib.variants(F32)] == [[128, 128, 32, 2, 32]]
    assert len({v[0] for dt in (F16, FP8, F32) for v in _lib.variants(dt)}) == 6
    assert L.wtc_list_variants(9, None, None, None, 0) == -1


# Shapes of the calibration sweep (welder_typical_chain_amd/calibrate.py)
# where the cost model picks the measured fastest (variant, path) on MI355X
# (back-to-back calls); tests/test_cost_model.py scores every shape.
MEASURED_BEST = [
    ((1, 2048, 2048, 1024, F16, F16), LDR[F16], _lib.PATH_EXCHANGE),   # C2: 14.6 vs 16.4 us
    ((1, 2048, 2048, 64, F16, F16), T128[F16], _lib.PATH_EXCHANGE),    # 8.1 vs 8.5
    ((1, 2048, 2048, 256, F16, F16), T128[F16], _lib.PATH_EXCHANGE),   # 9.2 vs 9.4
    ((1, 8192, 128, 64, F16, F16), T128[F16], _lib.PATH_EXCHANGE),     # 5.7 vs 5.8
    ((1, 4096, 4096, 1024, F16, F16), W256[F16], _lib.PATH_SPLIT),     # 52.5 vs 64.2
    ((1, 2048, 8192, 512, F16, F16), W256[F16], _lib.PATH_SPLIT),      # 40.1 vs 47.6
    ((8, 2048, 2048, 128, F16, F16), ROWS, _lib.PATH_ROWS),            # 50.3 vs split 54.3
    ((16, 512, 512, 64, F16, F16), T128[F16], _lib.PATH_EXCHANGE),     # 7.5 vs 8.0
    ((1, 4096, 2048, 128, F16, F16), T256[F16], _lib.PATH_SPLIT),      # 22.2 vs 24.4
    ((64, 2048, 2048, 128, F16, F16), ROWS, _lib.PATH_ROWS),           # C3: 250 vs 454
    ((1, 1024, 32768, 4096, BF16, BF16), W256[BF16], _lib.PATH_SPLIT),  # C4: 257 vs 293
    ((1, 8192, 8192, 4096, FP8, F16), W256[FP8], _lib.PATH_SPLIT),     # C5: 258 vs 347
]


@pytest.mark.parametrize("shape,tiles,path", MEASURED_BEST)
def test_model_picks_the_measured_fastest_variant(shape, tiles, path):
    pl = _lib.plan(*shape, _lib.PATH_AUTO)
    assert (pl["tiles"], pl["path"]) == (tiles, path)


def test_auto_is_the_first_of_the_ranking(L):
    """AUTO and an explicit path both take the variant with the lowest
    estimate among those that can run it; an explicit variant keeps its tiles."""
    shape = (1, 1152, 32768, 4096, BF16, BF16)
    best = _lib.plan(*shape, _lib.PATH_AUTO)
    ests = []
    for name, tiles, mask in _lib.variants(BF16):
        for p in (_lib.PATH_EXCHANGE, _lib.PATH_SPLIT, _lib.PATH_ROWS):
            if mask & (1 << p):
                try:
                    ests.append((_lib.plan(*shape, p, tiles)["est_us"], tiles, p))
                except _lib.WtcError:
                    pass
    est, tiles, p = min(ests)
    assert (best["tiles"], best["path"]) == (tiles, p) and abs(best["est_us"] - est) < 1e-9
    pinned = _lib.plan(*shape, _lib.PATH_SPLIT, T128[BF16])
    assert pinned["tiles"] == T128[BF16] and pinned["grid"] == 9 * 256


def test_variant_path_errors(L):
    # the 256-row variant runs no exchange path; rows needs k <= 128
    with pytest.raises(_lib.WtcError) as ei:
        _lib.plan(1, 512, 512, 64, F16, F16, _lib.PATH_EXCHANGE, T256[F16])
    assert ei.value.code == _lib.WTC_ERR_UNSUPPORTED and "does not run the exchange" in str(ei.value)
    with pytest.raises(_lib.WtcError) as ei:
        _lib.plan(1, 512, 512, 256, F16, F16, _lib.PATH_ROWS, ROWS)
    assert "k <= 128" in str(ei.value)
    # 16-bit tiles are no variant for fp8 (its k-tile holds 128 elements); the
    # unfused path has no rows variant
    with pytest.raises(_lib.WtcError) as ei:
        _lib.plan(1, 512, 512, 128, FP8, F16, _lib.PATH_AUTO, T128[F16])
    assert "no gfx950 kernel variant" in str(ei.value) and "256x128x128/2x32" in str(ei.value)
    with pytest.raises(_lib.WtcError):
        _lib.plan(1, 512, 512, 64, F16, F16, _lib.PATH_UNFUSED, ROWS)
    # an explicit variant with AUTO runs its own best path
    assert _lib.plan(1, 512, 512, 64, F16, F16, _lib.PATH_AUTO, T256[F16])["path"] == _lib.PATH_SPLIT
    assert _lib.plan(1, 512, 512, 64, F16, F16, _lib.PATH_AUTO, ROWS)["path"] == _lib.PATH_ROWS


@pytest.mark.parametrize("args,code", [
    ((1, 128, 128, 4, 1, 1, 0), _lib.WTC_ERR_ARG),     # k*2 bytes not a multiple of 16
    ((1, 128, 100, 64, 1, 1, 0), _lib.WTC_ERR_ARG),    # n not a multiple of 8
    ((1, -1, 128, 64, 1, 1, 0), _lib.WTC_ERR_ARG),
    ((1, 128, 128, 64, 7, 1, 0), _lib.WTC_ERR_ARG),    # in dtype
    ((1, 128, 128, 64, 1, 3, 0), _lib.WTC_ERR_ARG),    # fp8 output is not offered
    ((1, 128, 128, 64, 1, 1, 9), _lib.WTC_ERR_ARG),    # path
])
def test_plan_rejects_bad_arguments(L, args, code):
    rc, *_ = plan(L, *args)
    assert rc == code
    assert L.wtc_last_error()
    assert L.wtc_matmul_softmax_workspace_size(*args) < 0


def test_launch_argument_errors_without_gpu(L):
    # argument checks come before any HIP call
    rc = L.wtc_matmul_softmax(None, None, None, 1, 128, 128, 4, 1, 1, 1.0, 1.0, 1.0, 0, None, 0, None)
    assert rc == _lib.WTC_ERR_ARG
    # nothing to do: returns OK without touching a device
    rc = L.wtc_matmul_softmax(None, None, None, 1, 0, 128, 64, 1, 1, 1.0, 1.0, 1.0, 0, None, 0, None)
    assert rc == _lib.WTC_OK
    assert L.wtc_read_error_flags(None, None, 1) == _lib.WTC_ERR_ARG


# ---- compile / solver entry points --------------------------------------------

def write_chain(tmp_path: Path, cfg: ChainConfig, **kw) -> Path:
    p = tmp_path / f"{cfg.name.lower()}{'_named' if kw.get('named_softmax') else ''}.mlir"
    p.write_text(chain_mlir(cfg, **kw))
    return p


def solve(L, path: Path, out: Path, errsize=4096):
    tiles = [ctypes.c_int64() for _ in range(5)]
    err = ctypes.create_string_buffer(errsize) if errsize else None
    rc = L.welder_solver_solve_typical_chain(
        str(path).encode(), str(out / "best_summary.json").encode(),
        str(out / "candidates.tsv").encode(), 1, 0, *[ctypes.byref(t) for t in tiles], err, errsize)
    return rc, [t.value for t in tiles], (err.value if err is not None else b"")


def compile_chain(L, path: Path, out: Path, tiles, fused=1, errsize=4096):
    err = ctypes.create_string_buffer(errsize)
    rc = L.welder_compile_typical_chain_to_nvvm(str(path).encode(), str(out).encode(), b"", b"",
                                                *tiles, 1, fused, 0, err, errsize)
    return rc, err.value


EXPECT = {  # config -> (tiles of the variant the solver ranks first, its path)
    "C1": ([128, 128, 32, 2, 32], "exchange"), "C2": (LDR[F16], "exchange"), "C3": (ROWS, "rows"),
    "C4": (W256[BF16], "split"), "C5": (W256[FP8], "split"),
}


@pytest.mark.parametrize("name", sorted(EXPECT))
@pytest.mark.parametrize("named", [False, True])
def test_solver_and_compile_per_config(L, tmp_path, name, named):
    cfg = CONFIGS[name]
    src = write_chain(tmp_path, cfg, named_softmax=named)
    rc, tiles, err = solve(L, src, tmp_path)
    assert rc == 0, err
    want, path = EXPECT[name]
    assert tiles == want
    summary = json.loads((tmp_path / "best_summary.json").read_text())
    assert {k: summary["problem"][k] for k in "mnk"} == {"m": cfg.m, "n": cfg.n, "k": cfg.k}
    assert {"smemBytes", "numSM", "warpSize", "elementBytes"} <= set(summary["arch"])
    assert {"tileM", "tileN", "tileK", "threadTileM", "threadTileN", "score", "estimatedLatency",
            "profiledMs", "bytesCut"} <= set(summary["best"])
    rows = (tmp_path / "candidates.tsv").read_text().strip().split("\n")
    assert rows[0].split("\t") == ["rank", "tileM", "tileN", "tileK", "threadTileM", "threadTileN",
                                   "score", "estimatedLatency", "profiledMs", "bytesA", "bytesB",
                                   "bytesC", "bytesCut"]
    assert all(len(r.split("\t")) == 13 for r in rows[1:]) and len(rows) >= 2
    # bytesA: A is streamed once per column tile of the candidate's own width
    # (256 for the 256x256 tile, 128 otherwise); the rows path reads A once
    isz = {"f16": 2, "bf16": 2, "fp8": 1, "f32": 4}[cfg.in_dtype]
    a_bytes = cfg.batch * cfg.m * cfg.k * isz
    for r in rows[1:]:
        f = r.split("\t")
        tile_n, bytes_a = int(f[2]), int(f[9])
        assert bytes_a in (a_bytes, a_bytes * -(-cfg.n // tile_n)), (f, a_bytes)
        if tile_n == 256:
            assert bytes_a == a_bytes * -(-cfg.n // 256), f
    # the reference reads tiles from JSON with a first-match regex (Search.cpp:12-20)
    text = (tmp_path / "best_summary.json").read_text()
    got = [int(re.search(rf'"{k}"\s*:\s*(-?[0-9]+)', text).group(1))
           for k in ("tileM", "tileN", "tileK", "threadTileM", "threadTileN")]
    assert got == tiles

    out = tmp_path / "fused"
    rc, err = compile_chain(L, src, out, tiles)
    assert rc == 0, err
    launch = json.loads((out / "05.out.hip.launch.json").read_text())
    assert launch["problem"]["m"] == cfg.m and launch["problem"]["n"] == cfg.n
    assert launch["path"] == path and launch["entry"] == "wtc_matmul_softmax_tiles"
    assert [launch["tiles"][k] for k in ("tileM", "tileN", "tileK", "threadTileM",
                                         "threadTileN")] == tiles
    assert launch["runtime_scales"] == (cfg.in_dtype == "fp8")
    assert abs(launch["logit_scale"] - cfg.logit_scale) < 1e-6
    plan_json = json.loads((out / "04.kernel.plan.json").read_text())
    wide = tiles[:2] == [256, 256]
    assert plan_json["kernels"][0]["name"].startswith(
        "chain_rows_kernel" if path == "rows" else ("chain_wide_kernel" if wide else "chain_tile_kernel"))
    # rows kernel: 8 compute waves + 4 I/O waves; 256x256 tile and f32: 4 waves
    want_block = 768 if path == "rows" else (256 if cfg.in_dtype == "f32" or wide else 512)
    assert plan_json["kernels"][0]["block"][0] == want_block
    report = dict(l.split("=", 1) for l in (out / "kernel_report.txt").read_text().splitlines()
                  if "=" in l and " " not in l.split("=", 1)[0])
    assert int(report["launch_kernel_count"]) == (2 if path == "split" else 1)
    assert int(report["mfma_instruction_count"]) > 0
    assert int(report["scratch_instruction_count"]) == 0 and int(report["vgpr_spill_count"]) == 0
    assert int(report["kernels_without_resource_record"]) == 0
    assert (out / "05.out.gfx950.hsaco").stat().st_size > 0
    # the canonical chain written in stage 03 is itself a valid input
    out2 = tmp_path / "again"
    rc, err = compile_chain(L, out / "03.chain.canonical.mlir", out2, tiles)
    assert rc == 0, err
    again = json.loads((out2 / "05.out.hip.launch.json").read_text())
    assert again.pop("softmax_form") == "decomposed"
    launch.pop("softmax_form")
    assert again == launch


def test_compile_unfused_baseline(L, tmp_path):
    src = write_chain(tmp_path, CONFIGS["C2"])
    rc, err = compile_chain(L, src, tmp_path / "baseline", [128, 128, 64, 2, 16], fused=0)
    assert rc == 0, err
    plan_json = json.loads((tmp_path / "baseline" / "04.kernel.plan.json").read_text())
    assert [k["name"].split("<")[0] for k in plan_json["kernels"]] == [
        "chain_tile_kernel", "rowmax_kernel", "expsub_kernel", "rowsum_kernel", "rowdiv_kernel"]
    assert (tmp_path / "baseline" / "05.out.rows.gfx950.hsaco").exists()


def test_compile_error_codes(L, tmp_path):
    src = write_chain(tmp_path, CONFIGS["C2"])
    assert compile_chain(L, src, tmp_path / "o", [0, 128, 64, 2, 16])[0] == 1
    err = ctypes.create_string_buffer(64)
    assert L.welder_compile_typical_chain_to_nvvm(b"", b"x", b"", b"", 128, 128, 64, 2, 16, 1, 1, 0,
                                                  err, 64) == 1
    assert err.value
    rc, msg = compile_chain(L, src, tmp_path / "o", [64, 64, 64, 2, 16])  # no such variant
    assert rc == 2 and b"no gfx950 kernel variant" in msg
    bad = tmp_path / "bad.mlir"
    bad.write_text("module { func.func @main() { return } }")
    rc, msg = compile_chain(L, bad, tmp_path / "o", [128, 128, 64, 2, 16])
    assert rc == 2 and msg
    rc, msg = compile_chain(L, tmp_path / "missing.mlir", tmp_path / "o", [128, 128, 64, 2, 16])
    assert rc == 2


def test_solver_error_codes_and_truncation(L, tmp_path):
    src = write_chain(tmp_path, CONFIGS["C2"])
    tiles = [ctypes.c_int64() for _ in range(5)]
    err = ctypes.create_string_buffer(8)
    rc = L.welder_solver_solve_typical_chain(b"", b"a", b"b", 1, 0, *[ctypes.byref(t) for t in tiles],
                                             err, 8)
    assert rc == 1 and len(err.value) == 7  # truncated, NUL-terminated
    bad = tmp_path / "bad.mlir"
    bad.write_text("not mlir")
    assert solve(L, bad, tmp_path)[0] == 2
    (tmp_path / "plain_file").write_text("x")  # parent directories are created, but not through a file
    rc, _, msg = solve(L, src, tmp_path / "plain_file" / "dir")
    assert rc == 4 and msg
    assert solve(L, src, tmp_path, errsize=0)[0] == 0  # NULL error buffer is allowed


@pytest.mark.skipif(not REF_MLIR.exists(), reason="reference chain files not present")
@pytest.mark.parametrize("fname,expect", [
    ("matmul_softmax_chain.mlir", None),
    ("matmul_softmax_chain_f16_native.mlir", (8192, 128, 64, "f16")),
    ("matmul_softmax_chain_named_softmax.mlir", (8192, 128, 64, "f32")),
])
def test_reference_chain_files(L, tmp_path, fname, expect):
    src = REF_MLIR / fname
    rc, tiles, err = solve(L, src, tmp_path)
    assert rc == 0, err
    rc, err = compile_chain(L, src, tmp_path / "out", tiles)
    assert rc == 0, err
    launch = json.loads((tmp_path / "out" / "05.out.hip.launch.json").read_text())
    if expect:
        m, n, k, dt = expect
        assert (launch["problem"]["m"], launch["problem"]["n"], launch["problem"]["k"]) == (m, n, k)
        assert launch["in_dtype"] == dt


def test_one_hip_runtime_whichever_loads_first():
    """Loading the library before torch must not map a second HIP runtime."""
    import subprocess
    import sys
    code = ("from welder_typical_chain_amd import _lib; _lib.lib(); import torch, os; "
            "m = open(f'/proc/{os.getpid()}/maps').read().splitlines(); "
            "print(len({l.split()[-1] for l in m if 'libamdhip64' in l}))")
    out = subprocess.run([sys.executable, "-c", code], cwd=str(PKG.parent), capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "1"


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
@pytest.mark.parametrize("fused", [1, 0])
def test_compile_output_passes_reference_callers(L, tmp_path, name, fused):
    """Replays what the reference's callers do with an unmodified compile
    output directory: BuildCutEdgesTransform requires 05.out.nvvm.runnable.mlir
    (compiler/transform/BuildCutEdgesTransform.cpp:34,50-53), and
    validatePostbufferizeArtifacts requires 03.after_postbufferize.mlir,
    04.after_workgroup_launch.mlir and 05.out.nvvm.runnable.mlir to exist and
    be non-empty, then counts operations in them
    (compiler/runtime/PostbufferizeFixups.cpp:46-82)."""
    cfg = CONFIGS[name]
    src = write_chain(tmp_path, cfg)
    rc, tiles, err = solve(L, src, tmp_path)
    assert rc == 0, err
    out = tmp_path / ("fused" if fused else "baseline")
    rc, err = compile_chain(L, src, out, tiles, fused=fused)
    assert rc == 0, err
    # BuildCutEdgesTransform.cpp:34,50-53
    assert (out / "05.out.nvvm.runnable.mlir").exists()
    # PostbufferizeFixups.cpp:46-60
    post = (out / "03.after_postbufferize.mlir").read_text()
    launch = (out / "04.after_workgroup_launch.mlir").read_text()
    runnable = (out / "05.out.nvvm.runnable.mlir").read_text()
    assert post and launch and runnable
    # the counts the validator reports (PostbufferizeFixups.cpp:62-82)
    plan_json = json.loads((out / "04.kernel.plan.json").read_text())
    assert post.count("linalg.matmul") + post.count("linalg.batch_matmul") >= 1
    assert launch.count("gpu.launch") == len(plan_json["kernels"])
    assert launch.count("memref.alloca") == 0
    assert runnable.count("nvvm.mma.sync") == 0
    assert runnable.count("ld.local") == 0 and runnable.count("st.local") == 0
    # the launch plan module names each kernel's grid / block / LDS
    for k in plan_json["kernels"]:
        assert f"arith.constant {k['grid'][0]} : index" in launch
        assert f"arith.constant {k['block'][0]} : index" in launch
    assert f'wtc.path = "{plan_json["path"]}"' in runnable
    # bench/pin_baseline.sh:44-51 copies 03 / 04 / 04c / 05 of both variants
    # under `set -euo pipefail`: every one must exist
    for name in ("03.after_postbufferize.mlir", "04.after_workgroup_launch.mlir",
                 "04c.after_linalg_to_loops.mlir", "05.out.nvvm.runnable.mlir"):
        assert (out / name).is_file() and (out / name).stat().st_size > 0, name
    # bench/run_regression.sh:96-98,111-112 greps these patterns
    assert re.search(r"workgroup\(", launch)
    assert re.search(r"gpu\.launch_func", runnable)
    assert runnable.count("gpu.launch_func") == len(plan_json["kernels"])
    # 04c: one func per kernel, its grid as the parallel loop bound
    loops = (out / "04c.after_linalg_to_loops.mlir").read_text()
    assert loops.count("func.func @kernel") == len(plan_json["kernels"])
    for k in plan_json["kernels"]:
        assert f"%grid = arith.constant {k['grid'][0]} : index" in loops
