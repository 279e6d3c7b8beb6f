#!/usr/bin/env python3
"""Headline benchmark: fused f16 Matmul -> row-Softmax on one MI355X.

Workload ("C2"): A[2048x1024] f16 x B[1024x2048] f16,
f32 accumulation, softmax over N=2048, f16 output; inputs N(0,1)/sqrt(K)
(synthetic, generated on the GPU).  A "step" is one call of the fused chain
(`wtc_matmul_softmax`, one kernel launch on the exchange path).  Inputs are
resident in HBM before timing starts; W untimed warmups, then K back-to-back
timed steps bracketed by device synchronisation, timed with HIP events on the
launch stream (the reference's own method, WelderProfiler.cpp:752-792).

Prints ONE JSON line.  `roofline` prices the kernel against dense f16 MFMA
peak (2.5 PFLOP/s); `traffic` comes from the committed rocprofv3 --pmc
summary of this same command (profiles/), or is null.  `cpu_baseline` times
the chain lowered to f32 loops (oracle/, the restatement of the reference's
mlir-opt CPU path) on a bounded sample of rows on this host.  `launch`
gives the single-launch figures: one call's GPU time on an idle stream, its
difference from the back-to-back time per call (the launch overhead for short
calls; negative for long ones, which run at a higher clock when alone), and
the host enqueue cost.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_F16_TFLOPS = 2500.0     # MI355X dense f16/bf16 MFMA
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=500,
                    help="untimed steps first (500 C2 steps, ~10 ms, bring the clocks to their "
                         "steady state; a 10-step warmup times the first loop 2-5 %% slow)")
    ap.add_argument("--path", default="auto", choices=["auto", "exchange", "split", "unfused", "rows"])
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="budget of the cpu_baseline sample (0 disables it); C3-C5 time a row "
                         "sample of batch 0 and extrapolate")
    ap.add_argument("--workload", default="C2", choices=["C2", "C3", "C4", "C5"],
                    help="C2 is the headline; C3-C5 are the other BASELINE.json configurations, "
                         "timed the same way (their cpu_baseline extrapolates a row sample)")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="also time the vendor GEMM alone (torch.matmul / bmm on hipBLASLt; fp8: "
                         "torch._scaled_mm) on the same inputs, as context (\"vendor_gemm\")")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="before the timed steps, run plain device copies of this many MiB "
                         "(the byte-count calibration for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


def host_info():
    """The host the CPU baseline runs on: nproc (processing units this process
    may use, as GNU nproc counts them), logical CPUs, CPU model (lscpu)."""
    import subprocess
    info = {"logical_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}
    try:
        info["nproc"] = int(subprocess.run(["nproc"], capture_output=True, text=True,
                                           timeout=10).stdout.strip())
    except (OSError, ValueError, subprocess.SubprocessError):
        info["nproc"] = info["affinity_cpus"]
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((ln.split(":", 1)[1].strip() for ln in out.splitlines()
                      if ln.startswith("Model name")), None)
    except (OSError, subprocess.SubprocessError):
        pass
    info["model"] = model
    return info


def cpu_baseline(a_host, b_host, n, k, budget_s):
    """The chain lowered to f32 loops (oracle/wtc_oracle.c built with ROCm's
    clang -O3 and LLVM OpenMP, the restatement of the reference's mlir-opt CPU
    path): C2 on all `nproc` cores (all 2048 rows when the budget allows, else
    a row sample), C2 on one core (a row sample, extrapolated), and C1 in
    full on one core and on all cores."""
    from oracle import oracle as O
    from welder_typical_chain_amd.configs import CONFIGS
    host = host_info()
    threads = max(1, host["nproc"])
    rows_total = a_host.shape[0]
    # calibration: one row per thread
    _, t_cal = O.cpu_chain_loops(a_host, b_host, 0, threads, threads, baseline=True)
    per_row_all = max(t_cal / threads, 1e-9)
    rows = min(rows_total, max(threads, int(budget_s / 2 / per_row_all) // threads * threads))
    _, secs = O.cpu_chain_loops(a_host, b_host, 0, rows, threads, baseline=True)
    tflops = 2.0 * rows * n * k / secs / 1e12
    _, t_one = O.cpu_chain_loops(a_host, b_host, 0, 1, 1, baseline=True)
    rows1 = min(rows_total, max(4, int(budget_s / 3 / max(t_one, 1e-9))))
    _, secs1 = O.cpu_chain_loops(a_host, b_host, 0, rows1, 1, baseline=True)
    # C1 in full (128 rows), median of repeated runs
    c1 = CONFIGS["C1"]
    inp = O.make_inputs(c1, seed=0)
    a1, b1 = inp.a[0], inp.b[0]
    c1_us = {}
    for label, th in (("single_thread", 1), ("all_cores", threads)):
        runs = sorted(O.cpu_chain_loops(a1, b1, 0, c1.m, th, baseline=True)[1] for _ in range(15))
        c1_us[label] = round(runs[len(runs) // 2] * 1e6, 1)
    return {"value": round(tflops, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": (f"C2 {'all' if rows == rows_total else rows} of {rows_total} rows "
                       f"(f32 i-j-k loops + max/exp/sum/div, OpenMP over rows on {threads} threads), "
                       f"{secs:.2f} s"),
            "compiler": "ROCm clang -O3 -fopenmp (LLVM CPU backend)",
            "host": host, "threads": threads,
            "single_thread": {"value": round(2.0 * rows1 * n * k / secs1 / 1e12, 6), "cores": 1,
                              "sample": f"C2 {rows1} rows, {secs1:.2f} s",
                              "c2_full_s_extrapolated": round(secs1 * rows_total / rows1, 2)},
            "c1_full_us": {**c1_us, "flop": c1.flops,
                           "problem": "C1 f32 128x128 . 128x128, uniform[-1,1], seed 0"}}


def cpu_baseline_sample(cfg, a_host, b_host, budget_s):
    """C3-C5: the same f32 loop nest (inputs widened to f32: fp8 decoded and
    scaled) on a sample of batch 0's first rows, on all `nproc` cores and on
    one core, each extrapolated linearly to the whole problem (batch x M
    rows), as labelled.  The logit scale is left out: it does not change
    the loops' time."""
    from oracle import oracle as O
    host = host_info()
    threads = max(1, host["nproc"])
    n, k = cfg.n, cfg.k
    rows_total = cfg.batch * cfg.m
    _, t_cal = O.cpu_chain_loops(a_host, b_host, 0, threads, threads, baseline=True)
    per_row_all = max(t_cal / threads, 1e-9)
    rows = min(cfg.m, max(threads, int(budget_s / 2 / per_row_all) // threads * threads))
    _, secs = O.cpu_chain_loops(a_host, b_host, 0, rows, threads, baseline=True)
    _, t_one = O.cpu_chain_loops(a_host, b_host, 0, 1, 1, baseline=True)
    rows1 = min(cfg.m, max(2, int(budget_s / 3 / max(t_one, 1e-9))))
    _, secs1 = O.cpu_chain_loops(a_host, b_host, 0, rows1, 1, baseline=True)
    return {"value": round(2.0 * rows * n * k / secs / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": (f"{cfg.name} rows 0..{rows - 1} of batch 0 (f32 i-j-k loops + max/exp/sum/div, "
                       f"OpenMP over rows on {threads} threads), {secs:.2f} s"),
            "full_s_extrapolated": round(secs * rows_total / rows, 2),
            "compiler": "ROCm clang -O3 -fopenmp (LLVM CPU backend)", "host": host,
            "single_thread": {"value": round(2.0 * rows1 * n * k / secs1 / 1e12, 6), "cores": 1,
                              "sample": f"{cfg.name} {rows1} rows, {secs1:.2f} s",
                              "full_s_extrapolated": round(secs1 * rows_total / rows1, 2)}}


PEAKS = {"f16": PEAK_F16_TFLOPS, "bf16": PEAK_F16_TFLOPS, "fp8": 5000.0}
TORCH_DT = {"f16": "float16", "bf16": "bfloat16", "fp8": "float8_e4m3fn", "f32": "float32"}


def vendor_gemm(a, b, scale_a, scale_b, out_dtype, steps, torch):
    """The same product A.B alone (no softmax) through PyTorch's GEMM, which
    dispatches to hipBLASLt: torch.matmul (batched: bmm on contiguous
    operands), fp8 e4m3 through torch._scaled_mm with the per-tensor scales
    (its second operand column-major, as it requires).  HIP events over
    `steps` back-to-back calls after 20 warmups; context only."""
    if a.dtype == torch.float8_e4m3fn:
        bt = b.t().contiguous().t()
        sa = torch.tensor(scale_a, dtype=torch.float32, device=a.device)
        sb = torch.tensor(scale_b, dtype=torch.float32, device=a.device)
        op = "torch._scaled_mm (hipBLASLt, fp8 e4m3, per-tensor scales)"

        def f():
            return torch._scaled_mm(a, bt, scale_a=sa, scale_b=sb, out_dtype=out_dtype)
    elif a.dim() == 3:
        op = "torch.bmm (hipBLASLt)"

        def f():
            return torch.bmm(a, b)
    else:
        op = "torch.matmul (hipBLASLt)"

        def f():
            return torch.matmul(a, b)
    for _ in range(20):
        f()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        f()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    m, k = a.shape[-2], a.shape[-1]
    flops = 2 * (a.shape[0] if a.dim() == 3 else 1) * m * b.shape[-1] * k
    return {"op": op, "us_per_call": round(us, 2), "tflops": round(flops / (us * 1e-6) / 1e12, 1),
            "note": "the GEMM alone, without the softmax; context, not the metric"}


def make_workload(cfg, dev, torch):
    """Synthetic inputs of the configuration's distribution, generated on the GPU.
    Returns (a, b, logit_scale, scale_a, scale_b)."""
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    bshape = (cfg.batch,) if cfg.batch > 1 else ()
    sa = (*bshape, cfg.m, cfg.k)
    sb = (*bshape, cfg.k, cfg.n)
    if cfg.dist == "uniform":
        a32 = (torch.rand(sa, generator=g, device=dev) * 2 - 1) * cfg.dist_param
        b32 = (torch.rand(sb, generator=g, device=dev) * 2 - 1) * cfg.dist_param
    else:
        a32 = torch.randn(sa, generator=g, device=dev) * cfg.dist_param
        b32 = torch.randn(sb, generator=g, device=dev) * cfg.dist_param
    if cfg.in_dtype == "fp8":  # per-tensor amax scaling onto e4m3's range
        scale_a = float(a32.abs().max()) / 448.0
        scale_b = float(b32.abs().max()) / 448.0
        a = (a32 / scale_a).to(torch.float8_e4m3fn)
        b = (b32 / scale_b).to(torch.float8_e4m3fn)
    else:
        scale_a = scale_b = 1.0
        a = a32.to(getattr(torch, TORCH_DT[cfg.in_dtype]))
        b = b32.to(getattr(torch, TORCH_DT[cfg.in_dtype]))
    return a.contiguous(), b.contiguous(), cfg.logit_scale, scale_a, scale_b


# the path each committed traffic summary was measured on (what "auto" picks)
PROFILED_PATH = {"C2": "exchange", "C3": "rows", "C4": "split", "C5": "split"}


def load_traffic(workload: str = "C2", path: str = "auto"):
    """(HBM bytes per launch of the workload's dominant kernel, provenance)
    from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summaries.  The
    bytes are None if absent or if this run takes another path than the one
    profiled; the provenance names the summary, the source digest of the
    build it measured and of the build in this tree, so a stale figure shows."""
    from welder_typical_chain_amd.build import build_info
    this = build_info().get("source_digest")
    if path not in ("auto", PROFILED_PATH.get(workload)):
        return None, {"file": None, "this_build": this, "reason": "path not profiled"}
    name = "c2_f16_exchange_traffic.json" if workload == "C2" else "c3_c4_c5_traffic.json"
    try:
        doc = json.loads((ROOT / "profiles" / name).read_text())
        rec = doc if workload == "C2" else doc["workloads"][workload]
        built = doc.get("profile_build", {}).get("source_digest")
        return rec.get("hbm_bytes_per_launch"), {
            "file": f"profiles/{name}", "profile_build": built, "this_build": this,
            "same_build": built is not None and built == this}
    except (OSError, ValueError, KeyError):
        return None, {"file": None, "this_build": this, "reason": "no summary"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no "
              "multi-GPU path", file=sys.stderr)
        sys.exit(2)
    import torch
    from welder_typical_chain_amd import _lib
    from welder_typical_chain_amd.chain import matmul_softmax, new_workspace, workspace_size
    from welder_typical_chain_amd.configs import CONFIGS

    cfg = CONFIGS[args.workload]
    headline = args.workload == "C2"
    if not _lib.LIB_PATH.exists():
        from welder_typical_chain_amd import build
        build.build()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    m, n, k = cfg.m, cfg.n, cfg.k
    a, b, logit_scale, scale_a, scale_b = make_workload(cfg, dev, torch)
    out_dt = getattr(torch, TORCH_DT[cfg.out_dtype])
    out = torch.empty((*a.shape[:-2], m, n), dtype=out_dt, device=dev)
    in_code = {"f32": _lib.DTYPE_F32, "f16": _lib.DTYPE_F16, "bf16": _lib.DTYPE_BF16,
               "fp8": _lib.DTYPE_FP8_E4M3}[cfg.in_dtype]
    out_code = {"f32": _lib.DTYPE_F32, "f16": _lib.DTYPE_F16, "bf16": _lib.DTYPE_BF16}[cfg.out_dtype]
    ws = new_workspace(workspace_size(cfg.batch, m, n, k, in_code, out_code, args.path), dev)

    # One step = one call of the launcher C-ABI (the drop-in boundary), with
    # its arguments marshalled once: the torch wrapper's own host work (about
    # 5 us per call) would otherwise be timed too, and for short calls it,
    # not the GPU, sets the pace.  The first call goes through the wrapper,
    # which checks shapes and dtypes.
    matmul_softmax(a, b, out=out, path=args.path, workspace=ws, logit_scale=logit_scale,
                   scale_a=scale_a, scale_b=scale_b)
    launch = _lib.lib().wtc_matmul_softmax
    call_args = (a.data_ptr(), b.data_ptr(), out.data_ptr(), cfg.batch, m, n, k, in_code, out_code,
                 float(logit_scale), float(scale_a), float(scale_b), _lib.PATHS[args.path],
                 ws.data_ptr(), ws.numel(), torch.cuda.current_stream(dev).cuda_stream)

    def step():
        rc = launch(*call_args)
        if rc:
            _lib.check(rc)

    if args.copy_probe_mib > 0:
        n_el = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n_el, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t_host0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    t_host = time.perf_counter() - t_host0
    ms = e0.elapsed_time(e1) / args.steps

    # Single-launch figures, outside the timed region: the GPU time of one
    # call on an idle stream (events around it), its difference from the
    # back-to-back time per call, and the host's cost to enqueue one call.
    # The difference is the launch overhead for short calls; long calls
    # measured alone run at a higher clock than a sustained stream of them,
    # which makes it negative.
    single = []
    for _ in range(20):
        torch.cuda.synchronize()
        s0 = torch.cuda.Event(enable_timing=True)
        s1 = torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        step()
        s1.record(stream)
        s1.synchronize()
        single.append(s0.elapsed_time(s1) * 1e3)
    single_us = sorted(single)[len(single) // 2]
    torch.cuda.synchronize()
    h0 = time.perf_counter()
    for _ in range(50):
        step()
    enqueue_us = (time.perf_counter() - h0) / 50 * 1e6
    torch.cuda.synchronize()
    launch_info = {"single_call_us": round(single_us, 2), "back_to_back_us": round(ms * 1e3, 2),
                   "single_minus_back_to_back_us": round(single_us - ms * 1e3, 2),
                   "host_enqueue_us": round(enqueue_us, 2)}
    flops = cfg.flops
    tflops = flops / (ms * 1e-3) / 1e12
    from welder_typical_chain_amd.chain import read_error_flags
    flags = read_error_flags(ws)
    row_dev = float((out.float().sum(-1) - 1).abs().max()) if out.numel() <= (1 << 28) else \
        float((out[..., :256, :].float().sum(-1) - 1).abs().max())

    vendor = None
    if args.vendor_gemm:
        vendor = vendor_gemm(a, b, scale_a, scale_b, out_dt, min(args.steps, 50), torch)

    cpu = None
    if args.cpu_seconds > 0 and headline:
        cpu = cpu_baseline(a.float().cpu().numpy(), b.float().cpu().numpy(), n, k, args.cpu_seconds)
    elif args.cpu_seconds > 0:
        a0 = (a[0] if a.dim() == 3 else a).float() * scale_a
        b0 = (b[0] if b.dim() == 3 else b).float() * scale_b
        cpu = cpu_baseline_sample(cfg, a0.cpu().numpy(), b0.cpu().numpy(), args.cpu_seconds)
        del a0, b0

    peak = PEAKS[cfg.in_dtype]
    traffic, traffic_src = load_traffic(args.workload, args.path)
    alg_bytes = (a.numel() * a.element_size() + b.numel() * b.element_size() +
                 out.numel() * out.element_size())
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    if not headline:
        # HBM-bound when the arithmetic intensity is under the ridge point
        mfma_bound = flops / alg_bytes > peak * 1e12 / (PEAK_HBM_GBS * 1e9)
        line = {
            "metric": f"fused matmul+softmax TFLOP/s ({cfg.name})",
            "value": round(tflops, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "us_per_call": ms * 1e3,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": cfg.in_dtype, "data": f"synthetic {cfg.dist} inputs generated on the GPU",
            "config": {"workload": cfg.name, "batch": cfg.batch, "m": m, "n": n, "k": k,
                       "in_dtype": cfg.in_dtype, "out_dtype": cfg.out_dtype, "path": args.path},
            "roofline": ({"bound": "mfma", "achieved": round(tflops, 3), "peak": peak,
                          "unit": "TFLOP/s", "frac": round(tflops / peak, 4),
                          "traffic": traffic, "traffic_profile": traffic_src}
                         if mfma_bound else
                         {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                          "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                          "traffic": traffic, "traffic_profile": traffic_src}),
            "cpu_baseline": cpu,
            "launch": launch_info,
            "checks": {"row_sum_max_dev": row_dev, "device_error_flags": flags},
        }
        if vendor:
            line["vendor_gemm"] = vendor
        print(json.dumps(line), flush=True)
        return

    line = {
        "metric": "fused matmul+softmax TFLOP/s & % f16 MFMA peak (M=N=2048,K=1024)",
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "us_per_call": ms * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic N(0,1)/sqrt(K) f16 generated on the GPU",
        "config": {"workload": "C2 fused f16 matmul->row-softmax", "m": m, "n": n, "k": k,
                   "batch": 1, "accumulate": "f32", "out_dtype": "f16", "path": args.path},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": PEAK_F16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_F16_TFLOPS, 4),
                     "traffic": traffic, "traffic_profile": traffic_src},
        "cpu_baseline": cpu,
        "launch": launch_info,
        "checks": {"row_sum_max_dev": row_dev, "device_error_flags": flags,
                   "host_wall_s_timed_region": round(t_host, 4)},
    }
    if vendor:
        line["vendor_gemm"] = vendor
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
