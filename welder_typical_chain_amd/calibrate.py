"""Times every kernel variant on every path it runs, over a fixed set of
shapes, and prints one JSON line per (shape, variant, path) with the measured
and the modelled microseconds per call.

The constants of the cost model in csrc/variants.cpp are fitted to this
table (calibration_mi355x.jsonl holds the one they came from); after a
kernel change, measure again and refit:

    python -m welder_typical_chain_amd.calibrate [--set NAME] [--out FILE]
    python -m welder_typical_chain_amd.calibrate --fit FILE [FILE ...]

--fit prints the fitted constants and, for each shape set in turn, how well
a fit on the other sets ranks the variants of that one (the loss of the
model's pick against the measured fastest choice).

Each case: inputs N(0,1)/sqrt(K) (fp8: N(0,1) quantised), 10 untimed calls,
then back-to-back calls of the launcher C-ABI (arguments marshalled once)
between two HIP events on the launch stream, about 20 ms of GPU time.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import sys
import time

# name -> (batch, m, n, k, in dtype, out dtype)
SHAPES = {
    "c1_f32": (1, 128, 128, 128, "f32", "f32"),
    "f32_1k": (1, 1024, 1024, 1024, "f32", "f32"),
    "c2": (1, 2048, 2048, 1024, "f16", "f16"),
    "c2_k64": (1, 2048, 2048, 64, "f16", "f16"),
    "c2_k256": (1, 2048, 2048, 256, "f16", "f16"),
    "c2_k4096": (1, 2048, 2048, 4096, "f16", "f16"),
    "m1024": (1, 1024, 2048, 1024, "f16", "f16"),
    "m512": (1, 512, 2048, 1024, "f16", "f16"),
    "pinned": (1, 8192, 128, 64, "f16", "f16"),
    "sq4k": (1, 4096, 4096, 1024, "f16", "f16"),
    "n8k": (1, 2048, 8192, 512, "f16", "f16"),
    "big_f16": (1, 4096, 8192, 2048, "f16", "f16"),
    "attn8": (8, 2048, 2048, 128, "f16", "f16"),
    "attn16_small": (16, 512, 512, 64, "f16", "f16"),
    "rows_tall": (1, 4096, 2048, 128, "f16", "f16"),
    "c3": (64, 2048, 2048, 128, "f16", "f16"),
    "c4": (1, 1024, 32768, 4096, "bf16", "bf16"),
    "c5": (1, 8192, 8192, 4096, "fp8", "f16"),
    "fp8_c2": (1, 2048, 2048, 2048, "fp8", "f16"),
    "fp8_4k": (1, 4096, 4096, 2048, "fp8", "f16"),
}

# A second set, first held out; the constants are now fitted to both sets.
VALIDATION = {
    "v_sq3k": (1, 3072, 3072, 768, "f16", "f16"),
    "v_bf16_384t": (1, 1536, 4096, 1024, "bf16", "bf16"),
    "v_batch4": (4, 1024, 1024, 256, "f16", "f16"),
    "v_tall": (1, 6144, 2048, 512, "f16", "f16"),
    "v_attn32": (32, 1024, 1024, 64, "f16", "f16"),
    "v_n16k": (1, 2048, 16384, 1024, "bf16", "bf16"),
    "v_longk": (1, 512, 512, 4096, "f16", "f16"),
    "v_fp8_512t": (1, 2048, 4096, 4096, "fp8", "f16"),
    "v_attn128": (128, 1024, 1024, 128, "f16", "f16"),
    "v_tall16k": (1, 16384, 1024, 256, "f16", "f16"),
    "v_bf16_f32": (1, 2048, 2048, 512, "bf16", "f32"),
    "v_f32_2k": (1, 2048, 2048, 256, "f32", "f32"),
}

# Shapes the constants were not fitted to: the check that the fitted model
# still ranks the variants of unseen problems.
HOLDOUT = {
    "h_2560": (1, 2560, 2560, 1024, "f16", "f16"),
    "h_bf16_256t": (1, 1024, 4096, 2048, "bf16", "bf16"),
    "h_batch2": (2, 1536, 1536, 512, "f16", "f16"),
    "h_8k4k": (1, 8192, 4096, 512, "f16", "f16"),
    "h_attn48": (48, 1024, 1024, 128, "f16", "f16"),
    "h_attn4_k64": (4, 2048, 2048, 64, "f16", "f16"),
    "h_fp8_192t": (1, 3072, 1024, 2048, "fp8", "f16"),
    "h_fp8_n8k": (1, 1024, 8192, 1024, "fp8", "f16"),
    "h_640": (1, 640, 8192, 4096, "f16", "f16"),
    "h_f32_tall": (1, 4096, 512, 1024, "f32", "f32"),
    "h_n64k": (1, 256, 65536, 256, "bf16", "bf16"),
    "h_attn16_bf16": (16, 2048, 2048, 96, "bf16", "bf16"),
}

# More fp8 shapes and split-path shapes of several lengths of K, where the
# 256-row and 128-row variants are close.
EXTRA = {
    "e_fp8_2k8k_k512": (1, 2048, 8192, 512, "fp8", "f16"),
    "e_fp8_4k_k512": (1, 4096, 4096, 512, "fp8", "f16"),
    "e_fp8_4k8k_k1k": (1, 4096, 8192, 1024, "fp8", "f16"),
    "e_fp8_8k_k1k": (1, 8192, 8192, 1024, "fp8", "f16"),
    "e_fp8_2k_k8k": (1, 2048, 2048, 8192, "fp8", "f16"),
    "e_fp8_1k4k_k4k": (1, 1024, 4096, 4096, "fp8", "f16"),
    "e_fp8_8k4k_k2k": (1, 8192, 4096, 2048, "fp8", "f16"),
    "e_fp8_b4": (4, 1024, 2048, 2048, "fp8", "f16"),
    "e_fp8_1536": (1, 1536, 8192, 4096, "fp8", "f16"),
    "e_f16_4k_k256": (1, 4096, 4096, 256, "f16", "f16"),
    "e_f16_8k_k1k": (1, 8192, 8192, 1024, "f16", "f16"),
    "e_bf16_n32k_k1k": (1, 2048, 32768, 1024, "bf16", "bf16"),
    "e_f16_n16k_k4k": (1, 1024, 16384, 4096, "f16", "f16"),
    "e_bf16_4k_k4k": (1, 4096, 4096, 4096, "bf16", "bf16"),
    "e_f16_b2": (2, 2048, 4096, 1024, "f16", "f16"),
    "e_f16_3k4k": (1, 3072, 4096, 2048, "f16", "f16"),
}

PATH_NAMES = {1: "exchange", 2: "split", 3: "unfused", 4: "rows"}


def _set_of(name):
    for label, table in (("validation", VALIDATION), ("holdout", HOLDOUT), ("extra", EXTRA)):
        if name in table:
            return label
    return "fit"


def _inputs(batch, m, n, k, in_dt, device):
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(0)
    a = torch.randn((batch, m, k), generator=g, device=device) / math.sqrt(max(k, 1))
    b = torch.randn((batch, k, n), generator=g, device=device)
    if in_dt == "f32":
        return a, b
    if in_dt == "f16":
        return a.half(), b.half()
    if in_dt == "bf16":
        return a.bfloat16(), b.bfloat16()
    return (a * math.sqrt(max(k, 1))).to(torch.float8_e4m3fn), b.to(torch.float8_e4m3fn)


def time_case(shape, tiles, path, device, target_ms=20.0):
    """Mean microseconds per back-to-back call of one variant on one path."""
    import torch
    from . import _lib
    from .chain import new_workspace
    batch, m, n, k, in_dt, out_dt = shape
    codes = {"f32": _lib.DTYPE_F32, "f16": _lib.DTYPE_F16, "bf16": _lib.DTYPE_BF16,
             "fp8": _lib.DTYPE_FP8_E4M3}
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
    a, b = _inputs(batch, m, n, k, in_dt, device)
    out = torch.empty((batch, m, n), dtype=tdt[out_dt], device=device)
    ws_bytes = _lib.lib().wtc_matmul_softmax_workspace_size(batch, m, n, k, codes[in_dt],
                                                            codes[out_dt], path)
    ws = new_workspace(ws_bytes, device)
    t = _lib.Tiles(*tiles)
    stream = torch.cuda.current_stream(device)
    args = (a.data_ptr(), b.data_ptr(), out.data_ptr(), batch, m, n, k, codes[in_dt], codes[out_dt],
            1.0, 1.0, 1.0, ctypes.byref(t), path, ws.data_ptr(), ws.numel(), stream.cuda_stream)
    fn = _lib.lib().wtc_matmul_softmax_tiles

    def call():
        rc = fn(*args)
        if rc:
            _lib.check(rc)

    for _ in range(10):
        call()
    torch.cuda.synchronize(device)
    # a first estimate of the call time sets the number of timed calls
    t0 = time.perf_counter()
    for _ in range(5):
        call()
    torch.cuda.synchronize(device)
    est = (time.perf_counter() - t0) / 5 * 1e3
    iters = max(10, min(2000, int(target_ms / max(est, 1e-3))))
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(iters):
        call()
    e1.record(stream)
    torch.cuda.synchronize(device)
    us = e0.elapsed_time(e1) / iters * 1e3
    del a, b, out, ws
    return us, iters


# ---- fit --------------------------------------------------------------------------
# The cost model of csrc/variants.cpp for the fused paths (exchange, split,
# rows), with its constants as a vector; the C++ code holds the fitted
# values.

_VARIANT_IDS = {"tile128x128_wave64x32": 0, "tile128x128_wave64x64": 0,
                "tile128x128_wave64x64_loaders": 1, "tile256x128_wave64x64": 2,
                "rows128_wave64x32_k128": 3, "tile256x256_wave128x128": 4}
# tile rows and columns per tile variant id
_TILE = {0: (128, 128), 1: (128, 128), 2: (256, 128), 4: (256, 256)}
_IN_BYTES = {"f32": 4, "f16": 2, "bf16": 2, "fp8": 1}
_OUT_BYTES = {"f32": 4, "f16": 2, "bf16": 2}
# own k-tile cycles per (variant, input class 0 16-bit / 1 fp8 / 2 f32),
# fixed cycles per (variant, epilogue 0 exchange / 1 split), then scalars
_KT = [(0, 0), (0, 1), (0, 2), (1, 0), (1, 1), (2, 0), (2, 1), (4, 0), (4, 1)]
_FX = [(0, 0), (0, 1), (1, 0), (1, 1), (2, 1), (4, 1)]
_SCALARS = ["launch_us", "exchange_us", "exchange_per_tile_us", "hbm_gbs", "feed_gbs",
            "rows_block_cyc", "rows_tile_cyc", "rows_kstep_cyc"]


def _clock_ghz(busy):
    busy = min(1.0, max(0.0, busy))
    return 2.1 if busy <= 0.5 else 2.1 - 1.2 * (busy - 0.5)


def model_us(x, r, cu=256):
    """Modelled microseconds of one record (a fused path) for constants x."""
    kt = dict(zip(_KT, x[:len(_KT)]))
    fx = dict(zip(_FX, x[len(_KT):len(_KT) + len(_FX)]))
    c = dict(zip(_SCALARS, x[len(_KT) + len(_FX):]))
    b, m, n, k = r["batch"], r["m"], r["n"], r["k"]
    isz, osz = _IN_BYTES[r["in"]], _OUT_BYTES[r["out"]]
    v = _VARIANT_IDS[r["variant"]]
    elems = b * m * n
    ab = b * (m * k + k * n) * isz
    n_t = math.ceil(n / 128)
    us_per_byte = 1e6 / (c["hbm_gbs"] * 1e9)
    if v == 3:
        blocks = b * math.ceil(m / 128)
        waves = math.ceil(blocks / cu)
        f = _clock_ghz(blocks / (waves * cu))
        cyc = c["rows_block_cyc"] + n_t * (c["rows_tile_cyc"] + c["rows_kstep_cyc"] * math.ceil(k / 16))
        return c["launch_us"] + max(waves * cyc / (f * 1e3), (ab + elems * osz) * us_per_byte)
    rows, cols = _TILE[v]
    cls = 1 if r["in"] == "fp8" else (2 if r["in"] == "f32" else 0)
    n_t = math.ceil(n / cols)
    tiles = b * math.ceil(m / rows) * n_t
    waves = math.ceil(tiles / cu)
    f = _clock_ghz(tiles / (waves * cu))
    nk = math.ceil(k * isz / 128)
    epi = 0 if r["path"] == "exchange" else 1
    full, rem = tiles // cu, tiles % cu
    t_tiles = 0.0
    for count, active in ((full, cu), (1 if rem else 0, rem)):
        if count:
            per_kt = kt[(v, cls)] + (rows + cols) * 128 * active * f / c["feed_gbs"]
            t_tiles += count * (fx[(v, epi)] + nk * per_kt) / (f * 1e3)
    if r["path"] == "exchange":
        t_xch = c["exchange_us"] + c["exchange_per_tile_us"] * n_t if n > 128 else 0.0
        return c["launch_us"] + max(t_tiles, (ab + elems * osz) * us_per_byte) + t_xch
    stats = b * m * n_t * 8
    return (2 * c["launch_us"] + max(t_tiles, (ab + elems * osz + stats) * us_per_byte)
            + (2 * elems * osz + stats) * us_per_byte)


def fit_constants(records):
    """Least squares on log(model / measured) over the fused-path records."""
    import numpy as np
    from scipy.optimize import least_squares
    recs = [r for r in records if r["path"] != "unfused"]
    x0 = [800.0] * len(_KT) + [5000.0] * len(_FX) + [2.5, 1.0, 0.05, 6000.0, 60000.0, 3000.0,
                                                      5000.0, 100.0]
    lo = [0.0] * len(_KT) + [500.0] * len(_FX) + [0.5, 0.0, 0.0, 1000.0, 1000.0, 0.0, 0.0, 0.0]
    res = least_squares(lambda x: np.array([math.log(model_us(x, r) / r["us"]) for r in recs]),
                        np.maximum(x0, np.array(lo) + 1e-6), bounds=(lo, np.inf))
    return res.x


def ranking_losses(x, records):
    """Per shape: measured time of the model's pick over the measured best, - 1."""
    by = {}
    for r in records:
        if r["path"] != "unfused":
            by.setdefault(r["shape"], []).append(r)
    return {s: min(rs, key=lambda r: model_us(x, r))["us"] / min(r["us"] for r in rs) - 1
            for s, rs in by.items()}


def _report_fit(files):
    records = [json.loads(line) for f in files for line in open(f) if line.strip()]
    x = fit_constants(records)
    names = ([f"kt_cyc[variant {v}][class {c}]" for v, c in _KT] +
             [f"fixed_cyc[variant {v}][{'exchange' if e == 0 else 'split'}]" for v, e in _FX] +
             _SCALARS)
    for name, val in zip(names, x):
        print(f"{name:36s} {val:12.4f}")
    sets = sorted({r.get("set", "fit") for r in records})
    if len(sets) > 1:
        losses = []
        for held in sets:
            xs = fit_constants([r for r in records if r.get("set", "fit") != held])
            lo = ranking_losses(xs, [r for r in records if r.get("set", "fit") == held])
            losses += list(lo.values())
            print(f"held out {held:10s}: {len(lo)} shapes, mean loss {100 * sum(lo.values()) / len(lo):.2f} %, "
                  f"worst {100 * max(lo.values()):.1f} %")
        print(f"cross-validated: mean loss {100 * sum(losses) / len(losses):.2f} % over {len(losses)} shapes")
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", default=None, help="also write the JSON lines to this file")
    ap.add_argument("--shapes", default=None, help="comma-separated subset of the shape names")
    ap.add_argument("--set", choices=("fit", "validation", "holdout", "extra", "all"),
                    default="all", help="one of the shape sets, or all of them")
    ap.add_argument("--paths", default="exchange,split,rows,unfused")
    ap.add_argument("--fit", nargs="+", metavar="FILE", default=None,
                    help="fit the cost model's constants to these timing tables instead")
    args = ap.parse_args(argv)
    if args.fit:
        return _report_fit(args.fit)
    import torch
    from . import _lib
    device = torch.device("cuda", 0)
    cu = torch.cuda.get_device_properties(device).multi_processor_count
    table = {"fit": SHAPES, "validation": VALIDATION, "holdout": HOLDOUT, "extra": EXTRA,
             "all": {**SHAPES, **VALIDATION, **HOLDOUT, **EXTRA}}[args.set]
    names = args.shapes.split(",") if args.shapes else list(table)
    want_paths = {p for p, name in PATH_NAMES.items() if name in args.paths.split(",")}
    codes = {"f32": _lib.DTYPE_F32, "f16": _lib.DTYPE_F16, "bf16": _lib.DTYPE_BF16,
             "fp8": _lib.DTYPE_FP8_E4M3}
    sink = open(args.out, "w") if args.out else None
    for name in names:
        shape = table[name]
        batch, m, n, k, in_dt, out_dt = shape
        auto = _lib.plan(batch, m, n, k, codes[in_dt], codes[out_dt], _lib.PATH_AUTO, None, cu, 1)
        for vname, tiles, mask in _lib.variants(codes[in_dt]):
            for path in sorted(want_paths):
                if not mask & (1 << path):
                    continue
                try:
                    pl = _lib.plan(batch, m, n, k, codes[in_dt], codes[out_dt], path, tiles, cu, 1)
                except _lib.WtcError:
                    continue
                print(f"[calibrate] {name} {vname} {PATH_NAMES[path]}", file=sys.stderr, flush=True)
                us, iters = time_case(shape, tiles, path, device)
                rec = {"shape": name, "set": args.set if args.set != "all" else _set_of(name),
                       "batch": batch, "m": m, "n": n, "k": k, "in": in_dt,
                       "out": out_dt, "variant": vname, "tiles": tiles, "path": PATH_NAMES[path],
                       "grid": pl["grid"], "us": round(us, 3), "model_us": round(pl["est_us"], 3),
                       "iters": iters,
                       "auto": auto["tiles"] == tiles and auto["path"] == path}
                line = json.dumps(rec)
                print(line, flush=True)
                if sink:
                    sink.write(line + "\n")
                    sink.flush()
    if sink:
        sink.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
