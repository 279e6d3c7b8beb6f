"""Per-phase timeline of the exchange-path kernel (the C2 headline path),
from the phase stamps of the profiling build ``libwtc_hip_stamps.so``.

Every exchange tile's waves read the 100 MHz real-time counter at their
phase boundaries (layout in csrc/fused_matmul_softmax.hip); this script runs
back-to-back calls through that library's C-ABI, reads the stamps of the
last call of each round, and prints per-phase means / medians / maxima over
the tiles, the span of the kernel, the shader clock the tiles ran at, and the
mean time per call of each round (HIP events on the launch stream).

    python -m welder_typical_chain_amd.phase_timeline [--m 2048 --n 2048 --k 1024]
        [--warmup 500] [--rounds 5] [--calls 200] [--out FILE]

Needs a GPU and the built profiling library (python -m
welder_typical_chain_amd.build makes both libraries).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import sys

import numpy as np

from . import _lib

# (label, end word, start word, description); words of the stamp layout
PHASES = [
    ("first k-tile", 1, 0, "start -> k-tile 0 landed"),
    ("K loop", 2, 1, "k-tile 0 landed -> last k-tile's MFMAs issued and waited"),
    ("statistics", 3, 2, "row max / exp / sum of wave 0's block"),
    ("publish", 4, 3, "tile statistics combined, entries stored and acknowledged"),
    ("barrier A", 5, 4, "every wave past the publish"),
    ("stage tile", 6, 5, "MFMA wave 0 writes its f32 block to LDS"),
    ("loader poll", 14, 13, "first loader wave polls the row block's entries"),
    ("barrier B", 7, 6, "wave 0 waits for the table (the loaders' poll)"),
    ("merge", 8, 7, "row log-sum-exp from the table, factors to LDS"),
    ("barrier C", 9, 8, "factors in place, generation stored"),
    ("stores", 10, 9, "scale, convert, 16-byte stores, acknowledged"),
    ("tile total", 10, 0, "start -> stores acknowledged"),
]


def _stats(x: np.ndarray) -> tuple[float, float, float]:
    return float(x.mean()), float(np.median(x)), float(x.max())


def run(m: int, n: int, k: int, warmup: int, rounds: int, calls: int) -> dict:
    import torch
    L = _lib.stamps_lib()
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    a = (torch.randn((m, k), generator=g, device=dev) / math.sqrt(k)).half()
    b = torch.randn((k, n), generator=g, device=dev).half()
    out = torch.empty((m, n), dtype=torch.float16, device=dev)
    need = L.wtc_matmul_softmax_workspace_size(1, m, n, k, _lib.DTYPE_F16, _lib.DTYPE_F16,
                                               _lib.PATH_EXCHANGE)
    if need < 0:
        raise RuntimeError(L.wtc_last_error().decode())
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    s_ptr = stream.cuda_stream
    if L.wtc_workspace_init(ws.data_ptr(), need, s_ptr):
        raise RuntimeError(L.wtc_last_error().decode())
    grid = ctypes.c_int64()
    path = ctypes.c_int()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    if L.wtc_plan(1, m, n, k, _lib.DTYPE_F16, _lib.DTYPE_F16, _lib.PATH_EXCHANGE, cus, 1,
                  ctypes.byref(grid), ctypes.byref(path), None):
        raise RuntimeError(L.wtc_last_error().decode())
    tiles = int(grid.value)
    args = (a.data_ptr(), b.data_ptr(), out.data_ptr(), 1, m, n, k, _lib.DTYPE_F16, _lib.DTYPE_F16,
            1.0, 1.0, 1.0, _lib.PATH_EXCHANGE, ws.data_ptr(), need, s_ptr)

    def call():
        rc = L.wtc_matmul_softmax(*args)
        if rc:
            raise RuntimeError(L.wtc_last_error().decode())

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    buf = (ctypes.c_int64 * (tiles * 16))()
    per_round, stamps = [], []
    for r in range(rounds):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(calls):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        per_round.append(e0.elapsed_time(e1) * 1e3 / calls)
        if L.wtc_phase_stamps_read(buf, tiles):
            raise RuntimeError("wtc_phase_stamps_read failed")
        stamps.append(np.frombuffer(buf, dtype=np.int64).reshape(tiles, 16).copy())
        print(f"[phase_timeline] round {r + 1}/{rounds}: {per_round[-1]:.2f} us per call", flush=True)
    # the reference for the exact result: one more check that the stamps build computes the chain
    ref = torch.softmax(a[:64].float() @ b.float(), dim=-1)
    err = float((out[:64].float() - ref).abs().max())
    if not err < 2e-3:
        raise RuntimeError(f"stamps build output differs from the fp32 chain (max abs {err:.2e})")
    return {"m": m, "n": n, "k": k, "tiles": tiles, "us_per_call": per_round, "stamps": stamps}


def summarize(res: dict) -> str:
    st = np.concatenate(res["stamps"])  # [rounds * tiles, 16]
    rounds = len(res["stamps"])
    tiles = res["tiles"]
    us = lambda t: t / 100.0  # noqa: E731 - 100 MHz ticks to microseconds
    lines = [f"C2-shaped exchange kernel {res['m']}x{res['n']}x{res['k']} f16, {tiles} tiles, "
             f"last call of each of {rounds} rounds",
             "",
             f"us per call (HIP events, back-to-back rounds): "
             + ", ".join(f"{x:.2f}" for x in res["us_per_call"]),
             "",
             "| phase | mean us | median us | max us | what |",
             "|---|---|---|---|---|"]
    for label, end, start, what in PHASES:
        mean, med, mx = _stats(us(st[:, end] - st[:, start]))
        lines.append(f"| {label} | {mean:.2f} | {med:.2f} | {mx:.2f} | {what} |")
    spans, skews, arrive, clocks, kl_cycles = [], [], [], [], []
    nk = math.ceil(res["k"] * 2 / 128)  # 128-byte k-tiles of f16
    for s in res["stamps"]:
        t0 = s[:, 0].min()
        spans.append(us(s[:, 10].max() - t0))
        skews.append(us(s[:, 0].max() - t0))
        rb = s[:, 15] >> 8
        for r in np.unique(rb):
            pub = s[rb == r, 4]
            arrive.append(us(pub.max() - pub.min()))
        dt = (s[:, 2] - s[:, 1]).astype(np.float64)
        dc = (s[:, 12] - s[:, 11]).astype(np.float64)
        ok = dt > 0
        clocks.append(float(np.median(dc[ok] / dt[ok] * 0.1)))  # GHz
        kl_cycles.append(float(np.median(dc[ok] / max(nk - 1, 1))))
    lines += ["",
              "| kernel-wide | value |", "|---|---|",
              f"| span, first start to last store (us) | {np.mean(spans):.2f} "
              f"(rounds: {', '.join(f'{x:.2f}' for x in spans)}) |",
              f"| start skew, first to last tile (us) | {np.mean(skews):.2f} |",
              f"| row-block publish spread, mean / max (us) | {np.mean(arrive):.2f} / "
              f"{np.max(arrive):.2f} |",
              f"| shader clock over the K loop, median (GHz) | {np.mean(clocks):.2f} |",
              f"| K-loop cycles per k-tile, median | {np.mean(kl_cycles):.0f} |"]
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--m", type=int, default=2048)
    ap.add_argument("--n", type=int, default=2048)
    ap.add_argument("--k", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--rounds", type=int, default=5)
    ap.add_argument("--calls", type=int, default=200)
    ap.add_argument("--out", default=None, help="also write the table here")
    ap.add_argument("--json", default=None, help="raw stamps and per-round times as JSON")
    a = ap.parse_args(argv)
    res = run(a.m, a.n, a.k, a.warmup, a.rounds, a.calls)
    text = summarize(res)
    print(text, flush=True)
    if a.out:
        with open(a.out, "w") as f:
            f.write(text)
    if a.json:
        with open(a.json, "w") as f:
            json.dump({k: (v if k != "stamps" else [s.tolist() for s in v]) for k, v in res.items()}, f)
    return 0


if __name__ == "__main__":
    sys.exit(main())
