"""Fused-vs-unfused A/B harness for the Matmul -> row-Softmax chain.

The MI355X counterpart of the reference's bench/run_ab.sh (with
bench/run_compile_pair.sh, the welder-profiler perf / dump runs and
backend/welder/bench/verify_matmul_softmax.py behind it):

1. solve the tile parameters once (``welder_solver_solve_typical_chain``)
   and write ``search/best.json`` (the reference's compiler/scheduler/Search.cpp:76-81
   key set);
2. compile the chain twice with those tiles through
   ``welder_compile_typical_chain_to_nvvm``: fused=0 into ``baseline/``
   (the five-kernel unfused lowering), fused=1 into ``fused/``
   (bench/run_compile_pair.sh);
3. for each case, fill A and B with the profiler's input patterns
   (``zero`` / ``linear`` / ``random``, WelderProfilerRuntime.h:128-176),
   time ``iters`` back-to-back launches of the case's launch manifest after
   ``warmup`` untimed ones with HIP events on the launch stream
   (WelderProfiler.cpp:752-792), and append one row to ``ab_summary.tsv`` /
   ``ab_summary.csv`` with the header of bench/run_ab.sh:66-67;
4. with ``--verify``, run once more, dump the output (``out.bin`` plus the
   ``out.bin.json`` descriptor of WelderProfilerRuntime.h:104-126) and check
   sampled rows against a float64 recomputation with the pass rule
   ``|out - ref| <= atol + rtol * |ref|`` (verify_matmul_softmax.py:228-262);
5. write ``speedup.tsv`` = ``speedup\\t<baseline_ms / fused_ms, %.4f>``
   (bench/run_ab.sh:205-212).

Differences from the reference harness, each deliberate:
- inputs are quantised to the chain's element type with round-to-nearest-even
  (the profiler rounds f16 half-up, WelderProfilerEval.h:89; its own verifier
  uses RNE, verify_matmul_softmax.py:66-131);
- the baseline needs no ``--fill-each-iter``: every unfused kernel overwrites
  its whole intermediate, so no launch reads a value left by the previous one;
- rank-3 (batched) chains dump rank-3 descriptors; the descriptor also names
  the element type (``dtype``) because ``elem_bytes`` 2 covers f16 and bf16.

Usage: ``python -m welder_typical_chain_amd.run_ab [--input-mlir F | --m M --n N --k K]
[--out-base D] [--warmup 10] [--iters 200] [--pattern linear] [--seed 1] [--verify]``.
"""
from __future__ import annotations

import argparse
import csv
import ctypes
import json
import sys
from pathlib import Path

import numpy as np

_M32 = 0xFFFFFFFF
DEFAULT_ROWS = (0, 1, 2, 3, 7, 15, 31, 63, 127, 255, 511, 1023)
SUMMARY_HEADER = ("case", "avg_ms", "kernels", "pattern", "seed", "iters", "warmup", "out_dir")


# ---- input patterns (WelderProfilerRuntime.h:128-176) -------------------------

def _xorshift32(x: int) -> int:
    x ^= (x << 13) & _M32
    x ^= x >> 17
    x ^= (x << 5) & _M32
    return x & _M32


def _apply(cols: np.ndarray, x: np.ndarray) -> np.ndarray:
    """The GF(2)-linear map whose images of the 32 unit vectors are `cols`, applied to x."""
    out = np.zeros_like(x)
    for bit in range(32):
        out ^= ((x >> np.uint32(bit)) & np.uint32(1)) * cols[bit]
    return out


def xorshift32_states(n: int, seed: int) -> np.ndarray:
    """The first n states of the profiler's xorshift32 stream (seed 0 -> 1).

    The (13, 17, 5) shift-xor step is linear over GF(2), so the stream is built
    by doubling: with states s_1..s_h known and T^h as 32 column images,
    s_{h+1..2h} = T^h s_{1..h}, and T^2h = T^h T^h.  O(32 n) vector work.
    """
    out = np.empty(n, dtype=np.uint32)
    if n == 0:
        return out
    s = (seed & _M32) or 1
    out[0] = _xorshift32(s)
    cols = np.array([_xorshift32(1 << b) for b in range(32)], dtype=np.uint32)  # T^1
    have = 1
    while have < n:
        take = min(have, n - have)
        out[have:have + take] = _apply(cols, out[:take])
        cols = _apply(cols, cols)
        have += take
    return out


def pattern_values(pattern: str, n: int, seed: int) -> np.ndarray:
    """n float32 values of an input buffer in flat row-major order."""
    if pattern == "zero":
        return np.zeros(n, dtype=np.float32)
    if pattern == "linear":
        t = (np.arange(n, dtype=np.int64) % 1024).astype(np.float32)
        return t * np.float32(0.001) - np.float32(0.5)
    if pattern == "random":
        u = xorshift32_states(n, seed).astype(np.float32) * np.float32(1.0 / 4294967296.0)
        return u * np.float32(2.0) - np.float32(1.0)
    raise ValueError(f"unknown pattern {pattern!r} (zero, linear, random)")


# ---- dump format (WelderProfilerRuntime.h:104-126) ------------------------------

_ELEM_BYTES = {"f32": 4, "f16": 2, "bf16": 2}


def write_dump(path: Path, data: bytes, shape, dtype: str, sym: str = "%out") -> None:
    sizes = [int(s) for s in shape]
    strides = [int(np.prod(sizes[i + 1:])) for i in range(len(sizes))]
    Path(path).write_bytes(data)
    meta = {"sym": sym, "rank": len(sizes), "elem_bytes": _ELEM_BYTES[dtype], "offset": 0,
            "sizes": sizes, "strides": strides, "bytes": len(data), "dtype": dtype}
    Path(str(path) + ".json").write_text(json.dumps(meta, indent=2) + "\n")


def read_dump(path: Path):
    """(values as float64 ndarray shaped by `sizes`, descriptor dict)."""
    meta = json.loads(Path(str(path) + ".json").read_text())
    dtype = meta.get("dtype") or {4: "f32", 2: "f16"}[meta["elem_bytes"]]
    raw = Path(path).read_bytes()
    if len(raw) != meta["bytes"]:
        raise ValueError(f"{path}: {len(raw)} bytes, descriptor says {meta['bytes']}")
    if dtype == "f32":
        flat = np.frombuffer(raw, dtype="<f4").astype(np.float64)
    elif dtype == "f16":
        flat = np.frombuffer(raw, dtype="<f2").astype(np.float64)
    elif dtype == "bf16":
        flat = (np.frombuffer(raw, dtype="<u2").astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    else:
        raise ValueError(f"{path}: unsupported dump element type {dtype!r}")
    sizes, strides, off = meta["sizes"], meta["strides"], meta["offset"]
    view = np.lib.stride_tricks.as_strided(flat[off:], shape=sizes,
                                           strides=[s * 8 for s in strides])
    return np.array(view), meta


# ---- element-type rounding of the inputs ----------------------------------------

def quantize(x: np.ndarray, in_dtype: str) -> np.ndarray:
    """float32 values rounded to the chain's input type (RNE), returned as float32."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    dt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16,
          "fp8": torch.float8_e4m3fn}[in_dtype]
    return t.to(dt).to(torch.float32).numpy()


# ---- verifier (verify_matmul_softmax.py:134-272) ---------------------------------

def verify_dump(out_path: Path, *, k: int, pattern: str, seed: int, in_dtype: str,
                rtol: float, atol: float, logit_scale: float = 1.0,
                rows=DEFAULT_ROWS) -> tuple[bool, str]:
    """Sampled-row check of a dumped chain output against float64 softmax(scale * A.B).

    A and B are regenerated from (pattern, seed), each buffer restarting the
    stream as the profiler does, and rounded to in_dtype.  For a batched dump
    the rows are checked in the first and the last batch.
    """
    out, meta = read_dump(out_path)
    batched = out.ndim == 3
    batch = out.shape[0] if batched else 1
    m, n = out.shape[-2:]
    sel = [r for r in rows if 0 <= r < m]
    if not sel:
        return False, "FAIL: no valid rows selected"
    a = quantize(pattern_values(pattern, batch * m * k, seed), in_dtype).reshape(batch, m, k)
    b = quantize(pattern_values(pattern, batch * k * n, seed), in_dtype).reshape(batch, k, n)
    out3 = out.reshape(batch, m, n)
    max_abs = max_rel = 0.0
    ok = True
    for bi in sorted({0, batch - 1}):
        c = logit_scale * (a[bi, sel].astype(np.float64) @ b[bi].astype(np.float64))
        e = np.exp(c - c.max(axis=1, keepdims=True))
        ref = e / e.sum(axis=1, keepdims=True)
        got = out3[bi, sel]
        if not np.isfinite(got).all():
            return False, "FAIL: output contains NaN/Inf"
        diff = np.abs(got - ref)
        max_abs = max(max_abs, float(diff.max()))
        max_rel = max(max_rel, float((diff / np.maximum(np.abs(ref), 1e-6)).max()))
        ok &= bool((diff <= atol + rtol * np.abs(ref)).all())
    shape = f"({batch},{m},{n})" if batched else f"({m},{n})"
    msg = (f"{'PASS' if ok else 'FAIL'}: max_abs={max_abs:.6e} max_rel={max_rel:.6e} "
           f"shape={shape} rows={len(sel) * len({0, batch - 1})}")
    return ok, msg


# ---- solve / compile ---------------------------------------------------------------

def _err_buf():
    return ctypes.create_string_buffer(4096)


def solve_tiles(L, input_mlir: Path, search_dir: Path, max_connect_level: int = 1):
    search_dir.mkdir(parents=True, exist_ok=True)
    t = [ctypes.c_int64() for _ in range(5)]
    err = _err_buf()
    rc = L.welder_solver_solve_typical_chain(
        str(input_mlir).encode(), str(search_dir / "best_summary.json").encode(),
        str(search_dir / "candidates.tsv").encode(), max_connect_level, 0,
        *[ctypes.byref(x) for x in t], err, len(err))
    if rc != 0:
        raise RuntimeError(f"solver failed ({rc}): {err.value.decode(errors='replace')}")
    tiles = [int(x.value) for x in t]
    keys = ("tileM", "tileN", "tileK", "threadTileM", "threadTileN")
    (search_dir / "best.json").write_text(
        "{\n" + ",\n".join(f'  "{kk}": {v}' for kk, v in zip(keys, tiles)) + "\n}\n")
    return tiles


def compile_case(L, input_mlir: Path, out_dir: Path, tiles, fused: bool,
                 max_connect_level: int = 1) -> dict:
    out_dir.mkdir(parents=True, exist_ok=True)
    err = _err_buf()
    rc = L.welder_compile_typical_chain_to_nvvm(
        str(input_mlir).encode(), str(out_dir).encode(), b"", b"", *tiles,
        max_connect_level if fused else 0, 1 if fused else 0, 0, err, len(err))
    if rc != 0:
        raise RuntimeError(f"compile ({'fused' if fused else 'baseline'}) failed ({rc}): "
                           f"{err.value.decode(errors='replace')}")
    return json.loads((out_dir / "05.out.hip.launch.json").read_text())


def kernel_count(out_dir: Path) -> int:
    plan = json.loads((out_dir / "04.kernel.plan.json").read_text())
    return len(plan["kernels"])


# ---- one case: fill, time, optionally dump ------------------------------------------

_TORCH_IN = {"f32": "float32", "f16": "float16", "bf16": "bfloat16", "fp8": "float8_e4m3fn"}


def run_case(launch: dict, *, pattern: str, seed: int, warmup: int, iters: int,
             dump: Path | None = None, device: str = "cuda:0") -> float:
    """Average milliseconds per launch of the manifest's entry point (HIP events)."""
    import torch
    from .chain import matmul_softmax, new_workspace

    p = launch["problem"]
    batch, m, n, k = p["batch"], p["m"], p["n"], p["k"]
    batched = bool(p.get("batched")) or batch > 1
    in_dt, out_dt = launch["in_dtype"], launch["out_dtype"]
    lead = (batch,) if batched else ()
    a_host = quantize(pattern_values(pattern, batch * m * k, seed), in_dt).reshape(*lead, m, k)
    b_host = quantize(pattern_values(pattern, batch * k * n, seed), in_dt).reshape(*lead, k, n)
    dev = torch.device(device)
    tdt = getattr(torch, _TORCH_IN[in_dt])
    a = torch.from_numpy(a_host).to(dev).to(tdt).contiguous()
    b = torch.from_numpy(b_host).to(dev).to(tdt).contiguous()
    out = torch.empty((*lead, m, n), dtype=getattr(torch, _TORCH_IN[out_dt]), device=dev)
    ws = new_workspace(launch["workspace_bytes"], dev)
    path = launch["path"]
    scale = float(launch.get("logit_scale", 1.0))

    # The first call goes through the torch wrapper (shape / dtype checks); the
    # timed ones call the launcher C-ABI with its arguments marshalled once, as
    # the reference's profiler times back-to-back launches from C++
    # (WelderProfiler.cpp:752-792) without per-call host work of its own.
    # the manifest names the kernel variant (best.json's tiles) that runs
    tiles = [int(launch["tiles"][key]) for key in ("tileM", "tileN", "tileK", "threadTileM",
                                                   "threadTileN")]
    matmul_softmax(a, b, out=out, path=path, workspace=ws, logit_scale=scale, tiles=tiles)
    from . import _lib
    launch_fn = _lib.lib().wtc_matmul_softmax_tiles
    in_code = {"f32": _lib.DTYPE_F32, "f16": _lib.DTYPE_F16, "bf16": _lib.DTYPE_BF16,
               "fp8": _lib.DTYPE_FP8_E4M3}[in_dt]
    out_code = {"f32": _lib.DTYPE_F32, "f16": _lib.DTYPE_F16, "bf16": _lib.DTYPE_BF16}[out_dt]
    ctiles = _lib.Tiles(*tiles)
    call_args = (a.data_ptr(), b.data_ptr(), out.data_ptr(), batch, m, n, k, in_code, out_code,
                 scale, 1.0, 1.0, ctypes.byref(ctiles), _lib.PATHS[path], ws.data_ptr(),
                 ws.numel(), torch.cuda.current_stream(dev).cuda_stream)

    def step():
        rc = launch_fn(*call_args)
        if rc:
            _lib.check(rc)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(iters):
        step()
    e1.record(stream)
    torch.cuda.synchronize(dev)
    avg_ms = e0.elapsed_time(e1) / max(iters, 1)
    if dump is not None:
        host = out.view(torch.int16 if out.element_size() == 2 else torch.int32).cpu().numpy()
        write_dump(dump, host.tobytes(), out.shape, out_dt)
    return avg_ms


# ---- driver -----------------------------------------------------------------------

def _default_chain(args) -> Path:
    from .chain_mlir import chain_mlir
    from .configs import ChainConfig
    cfg = ChainConfig("ab", args.batch, args.m, args.n, args.k, args.in_dtype, args.out_dtype,
                      "uniform", 1.0, logit_scale=args.logit_scale)
    path = Path(args.out_base) / "input.mlir"
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(chain_mlir(cfg))
    return path


def run_ab(args) -> dict:
    from . import _lib
    L = _lib.lib()
    base = Path(args.out_base)
    base.mkdir(parents=True, exist_ok=True)
    src = Path(args.input_mlir) if args.input_mlir else _default_chain(args)
    if not src.is_file():
        raise SystemExit(f"error: input mlir not found: {src}")
    tiles = solve_tiles(L, src, base / "search", args.max_connect_level)
    tsv = open(base / "ab_summary.tsv", "w", newline="")
    cs = open(base / "ab_summary.csv", "w", newline="")
    tsv.write("\t".join(SUMMARY_HEADER) + "\n")
    cw = csv.writer(cs, lineterminator="\n")
    cw.writerow(SUMMARY_HEADER)
    results = {}
    verify_ok = {}
    try:
        for name, fused in (("baseline", False), ("fused", True)):
            out_dir = base / name
            launch = compile_case(L, src, out_dir, tiles, fused, args.max_connect_level)
            print(f"[run:{name}] perf", flush=True)
            ms = run_case(launch, pattern=args.pattern, seed=args.seed, warmup=args.warmup,
                          iters=args.iters)
            kernels = kernel_count(out_dir)
            (out_dir / "profile.log").write_text(
                f"path={launch['path']} kernels={kernels} warmup={args.warmup} iters={args.iters}\n"
                f"avg_ms={ms:.6f}\n")
            if args.verify:
                print(f"[run:{name}] verify", flush=True)
                dump = out_dir / "out.bin"
                run_case(launch, pattern=args.pattern, seed=args.seed, warmup=args.verify_warmup,
                         iters=args.verify_iters, dump=dump)
                ok, msg = verify_dump(dump, k=launch["problem"]["k"], pattern=args.pattern,
                                      seed=args.seed, in_dtype=launch["in_dtype"],
                                      rtol=args.verify_rtol, atol=args.verify_atol,
                                      logit_scale=float(launch.get("logit_scale", 1.0)))
                (out_dir / "verify.log").write_text(msg + "\n")
                print(msg, flush=True)
                if not ok:
                    print(f"[warn:{name}] numerical verification failed "
                          f"(see {out_dir / 'verify.log'})", flush=True)
                verify_ok[name] = ok
            row = (name, f"{ms:.6f}", kernels, args.pattern, args.seed, args.iters, args.warmup,
                   str(out_dir))
            tsv.write("\t".join(str(x) for x in row) + "\n")
            cw.writerow(row)
            results[name] = ms
            print(f"summary:{name}: avg_ms={ms:.6f} kernels={kernels} out_dir={out_dir}", flush=True)
    finally:
        tsv.close()
        cs.close()
    fused_ms = results["fused"]
    speedup = "nan" if fused_ms == 0 else f"{results['baseline'] / fused_ms:.4f}"
    (base / "speedup.tsv").write_text(f"speedup\t{speedup}\n")
    print(f"speedup\t{speedup}")
    print(f"done: baseline={base / 'baseline'} fused={base / 'fused'} speedup={speedup}x", flush=True)
    return {"baseline_ms": results["baseline"], "fused_ms": fused_ms, "speedup": speedup,
            "tiles": tiles, "verify": verify_ok}


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--input-mlir", default=None,
                    help="chain MLIR file (default: a generated chain of --m/--n/--k)")
    ap.add_argument("--out-base", default="/tmp/wtc_ab")
    ap.add_argument("--max-connect-level", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--verify", action="store_true")
    ap.add_argument("--verify-warmup", type=int, default=0)
    ap.add_argument("--verify-iters", type=int, default=1)
    ap.add_argument("--verify-rtol", type=float, default=1e-3)
    ap.add_argument("--verify-atol", type=float, default=1e-3)
    ap.add_argument("--pattern", default="linear", choices=["zero", "linear", "random"])
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--m", type=int, default=8192)
    ap.add_argument("--k", type=int, default=64)
    ap.add_argument("--n", type=int, default=128)
    ap.add_argument("--in-dtype", default="f16", choices=["f32", "f16", "bf16", "fp8"])
    ap.add_argument("--out-dtype", default="f32", choices=["f32", "f16", "bf16"])
    ap.add_argument("--logit-scale", type=float, default=1.0)
    return ap.parse_args(argv)


def main(argv=None) -> int:
    args = parse_args(argv)
    res = run_ab(args)
    return 0 if all(res["verify"].values()) else 1


if __name__ == "__main__":
    sys.exit(main())
