"""GPU parity of the HIP chain against the CPU oracle (through the C-ABI).

Every case prints its name before touching the GPU.  Tolerances are the ones
stated in tests/parity_util.py.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from welder_typical_chain_amd.configs import CONFIGS, ChainConfig  # noqa: E402

from .parity_util import (check_row_sums, compare_rows, logit_error_bound, run_chain,  # noqa: E402
                          sample_rows)

pytestmark = pytest.mark.gpu

needs_gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="no GPU")


def _announce(msg: str) -> None:
    print(f"\n[gpu-case] {msg}", flush=True)


def _check(cfg: ChainConfig, inp: O.ChainInputs, out: torch.Tensor, rows, batches=(0,),
           path: str = "auto"):
    out_np = out.float().cpu().numpy()
    if out_np.ndim == 2:
        out_np = out_np[None]
    metrics = []
    for bt in batches:
        logits, probs = O.chain_rows(inp.a[bt], inp.b[bt], rows, inp.scale)
        err = logit_error_bound(inp.a[bt], inp.b[bt], rows, inp.scale, logits, cfg.in_dtype)
        metrics.append(compare_rows(out_np[bt][rows], probs, logits, cfg.out_dtype,
                                    label=f"{cfg.name} batch {bt}", in_dtype=cfg.in_dtype, logit_err=err))
    # the split path (also what "auto" picks for C4 and C5) keeps an f16 intermediate
    split = path == "split" or (path == "auto" and cfg.name in ("C4", "C5"))
    check_row_sums(out, cfg.name, split=split)
    return metrics


@needs_gpu
def test_c1_f32_full(native_lib):
    cfg = CONFIGS["C1"]
    _announce("C1 f32 128x128x128 all rows")
    inp = O.make_inputs(cfg, seed=0)
    for path in ("auto", "exchange", "split", "unfused"):
        out = run_chain(inp, cfg.in_dtype, cfg.out_dtype, path=path)
        _check(cfg, inp, out, np.arange(cfg.m))


@needs_gpu
@pytest.mark.parametrize("path", ["auto", "exchange", "split", "unfused"])
def test_c2_f16_headline(native_lib, path):
    cfg = CONFIGS["C2"]
    _announce(f"C2 f16 2048x2048x1024 path={path}")
    inp = O.make_inputs(cfg, seed=0)
    out = run_chain(inp, cfg.in_dtype, cfg.out_dtype, path=path)
    _check(cfg, inp, out, sample_rows(cfg.m, 48))
    from welder_typical_chain_amd.chain import read_diagnostics
    flags, longest_wait, timeouts = read_diagnostics()
    print(f"[gpu-case] row-block waits: longest {longest_wait / 100:.1f} us, timeouts {timeouts}")
    assert flags == 0 and timeouts == 0


@needs_gpu
@pytest.mark.parametrize("in_dtype,out_dtype", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32"),
                                                ("fp8", "f16"), ("f32", "f32"), ("bf16", "f16")])
@pytest.mark.parametrize("path", ["exchange", "split"])
def test_ragged_shapes(native_lib, in_dtype, out_dtype, path):
    # M, N, K not multiples of the 128x128 tile / 128-byte k-tile
    m, n = 200, 264
    k = {"f16": 72, "bf16": 72, "f32": 36, "fp8": 80}[in_dtype]
    dist = "xorshift_uniform" if in_dtype == "f32" else "normal"
    cfg = ChainConfig("ragged", 1, m, n, k, in_dtype, out_dtype, dist, 0.3)
    _announce(f"ragged {in_dtype}->{out_dtype} {m}x{n}x{k} path={path}")
    inp = O.make_inputs(cfg, seed=3)
    out = run_chain(inp, in_dtype, out_dtype, path=path)
    _check(cfg, inp, out, np.arange(m), path=path)


@needs_gpu
@pytest.mark.parametrize("in_dtype,out_dtype", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32"),
                                                ("fp8", "f16"), ("f32", "f32"), ("bf16", "f16")])
@pytest.mark.parametrize("n", [128, 72])
def test_exchange_single_column_tile(native_lib, in_dtype, out_dtype, n):
    """N <= 128: one column tile per row block, normalised from the tile's own
    statistics without the cross-workgroup exchange (ragged M and K too), and
    the row-block counters are left untouched for the next call."""
    from welder_typical_chain_amd.chain import new_workspace, read_diagnostics, workspace_size
    m = 300
    k = {"f16": 72, "bf16": 72, "f32": 36, "fp8": 80}[in_dtype]
    dist = "xorshift_uniform" if in_dtype == "f32" else "normal"
    cfg = ChainConfig("solo", 1, m, n, k, in_dtype, out_dtype, dist, 0.3)
    _announce(f"single column tile {in_dtype}->{out_dtype} {m}x{n}x{k} path=exchange")
    codes = {"f32": 0, "f16": 1, "bf16": 2, "fp8": 3}
    ws = new_workspace(workspace_size(1, 2048, 2048, 1024, codes[in_dtype], codes[out_dtype]))
    inp = O.make_inputs(cfg, seed=9)
    out = run_chain(inp, in_dtype, out_dtype, path="exchange", workspace=ws)
    _check(cfg, inp, out, np.arange(m))
    # the same workspace then serves a multi-tile exchange call correctly
    cfg2 = ChainConfig("after-solo", 1, 256, 384, k, in_dtype, out_dtype, dist, 0.3)
    inp2 = O.make_inputs(cfg2, seed=10)
    out2 = run_chain(inp2, in_dtype, out_dtype, path="exchange", workspace=ws)
    _check(cfg2, inp2, out2, np.arange(256))
    flags, _, timeouts = read_diagnostics(ws)
    assert flags == 0 and timeouts == 0


@needs_gpu
@pytest.mark.parametrize("in_dtype,out_dtype", [("f16", "f16"), ("bf16", "f32"), ("fp8", "f16"),
                                                ("bf16", "bf16")])
def test_split_256_row_tiles_ragged(native_lib, in_dtype, out_dtype):
    """The split path's 256-row tile variant: batch 64 x 200 rows (56 padding
    rows in each tile), ragged N and K."""
    from welder_typical_chain_amd import _lib
    batch, m, n = 64, 200, 1000
    k = {"f16": 72, "bf16": 72, "fp8": 80}[in_dtype]
    codes = {"f16": 1, "bf16": 2, "fp8": 3, "f32": 0}
    tiles = [256, 128, 128 // (2 if in_dtype != "fp8" else 1), 2, 32]
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    pl = _lib.plan(batch, m, n, k, codes[in_dtype], codes[out_dtype], _lib.PATH_SPLIT, tiles, cu)
    assert pl["grid"] == batch * 1 * 8, "expected one 256-row tile per batch and column tile"
    cfg = ChainConfig("split256", batch, m, n, k, in_dtype, out_dtype, "normal", 0.4,
                      logit_scale=0.7)
    _announce(f"split 256-row tiles {in_dtype}->{out_dtype} {batch}x{m}x{n}x{k}")
    inp = O.make_inputs(cfg, seed=11)
    out = run_chain(inp, in_dtype, out_dtype, path="split", batched=True, tiles=tiles)
    _check(cfg, inp, out, np.arange(m), batches=(0, 31, 63), path="split")


@needs_gpu
@pytest.mark.parametrize("path", ["auto", "split"])
def test_c3_batched_attention(native_lib, path):
    cfg = CONFIGS["C3"]
    _announce(f"C3 f16 batched 8x2048x2048x128 (batch subset) path={path}")
    inp = O.make_inputs(cfg, seed=0, batch=8)
    out = run_chain(inp, cfg.in_dtype, cfg.out_dtype, path=path, batched=True)
    _check(cfg, inp, out, sample_rows(cfg.m, 8), batches=(0, 5, 7))


@needs_gpu
def test_c3_full_batch(native_lib):
    """C3 at its configured size: 64 batch x heads of 2048 x 2048 x 128, scale
    1/sqrt(128), through auto (the row-block path: 1024 row blocks, four per
    CU).  Sampled rows of batches 0, 31 and 63 against the oracle; the row
    sums of all 131072 rows on the GPU."""
    cfg = CONFIGS["C3"]
    _announce("C3 f16 batched 64x2048x2048x128 (full size) path=auto")
    inp = O.make_inputs(cfg, seed=0)
    assert inp.a.shape[0] == 64
    out = run_chain(inp, cfg.in_dtype, cfg.out_dtype, path="auto", batched=True)
    rows = sample_rows(cfg.m, 12)
    for bt in (0, 31, 63):
        logits, probs = O.chain_rows(inp.a[bt], inp.b[bt], rows, inp.scale)
        got = out[bt][torch.from_numpy(rows).to(out.device)].float().cpu().numpy()
        err = logit_error_bound(inp.a[bt], inp.b[bt], rows, inp.scale, logits, cfg.in_dtype)
        compare_rows(got, probs, logits, cfg.out_dtype, label=f"C3 batch {bt}", in_dtype=cfg.in_dtype,
                     logit_err=err)
    worst = 0.0
    for bt in range(0, 64, 8):  # row sums in chunks of 8 batches (16 Mi entries each)
        s = out[bt:bt + 8].float().sum(-1)
        worst = max(worst, float((s - 1.0).abs().max()))
        assert bool(torch.isfinite(out[bt:bt + 8]).all())
    print(f"[gpu-case] C3 full: max row-sum deviation {worst:.2e} over 131072 rows")
    assert worst <= 1e-3


@needs_gpu
def test_exchange_calls_on_two_streams(native_lib):
    """Exchange-path calls alternating between two streams with their own
    workspaces: the library orders them (each needs all of its tiles
    resident), so every result matches the fp32 reference and no wait times
    out."""
    import math
    from welder_typical_chain_amd.chain import (check_status, matmul_softmax, new_workspace,
                                                read_diagnostics, workspace_size)
    _announce("exchange calls alternating between two streams, 2 x 12 calls")
    dev = torch.device("cuda")
    m = n = 2048
    k = 512
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    wss = [new_workspace(workspace_size(1, m, n, k, 1, 1, "exchange"), dev) for _ in streams]
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    jobs = []
    for it in range(24):
        a = (torch.randn((m, k), generator=g, device=dev) / math.sqrt(k)).half()
        b = (torch.randn((k, n), generator=g, device=dev) * (1 + it / 12)).half()
        jobs.append((a, b))
    torch.cuda.synchronize()
    outs = []
    for it, (a, b) in enumerate(jobs):
        i = it % 2
        streams[i].wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(streams[i]):
            outs.append(matmul_softmax(a, b, path="exchange", workspace=wss[i]))
    torch.cuda.synchronize()
    check_status()
    worst = 0.0
    for (a, b), out in zip(jobs, outs):
        ref = torch.softmax(a.float() @ b.float(), dim=-1)
        worst = max(worst, float((out.float() - ref).abs().max()))
    flags = [read_diagnostics(w) for w in wss]
    print(f"[gpu-case] worst abs err {worst:.2e}; diagnostics {flags}")
    assert worst < 2e-3 and all(f[0] == 0 and f[2] == 0 for f in flags)


@needs_gpu
@pytest.mark.parametrize("in_dtype,out_dtype", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32"),
                                                ("bf16", "f16")])
@pytest.mark.parametrize("m,n,k", [(200, 264, 72), (128, 128, 128), (64, 4104, 8), (300, 136, 120),
                                   (128, 384, 128), (300, 520, 120)])
def test_rows_path_shapes(native_lib, in_dtype, out_dtype, m, n, k):
    """The one-workgroup-per-row-block path: ragged M / N, K below the
    k-step, a wide row of many column tiles."""
    cfg = ChainConfig("rows", 1, m, n, k, in_dtype, out_dtype, "normal", 0.4, logit_scale=0.6)
    _announce(f"rows path {in_dtype}->{out_dtype} {m}x{n}x{k}")
    inp = O.make_inputs(cfg, seed=5)
    out = run_chain(inp, in_dtype, out_dtype, path="rows")
    _check(cfg, inp, out, np.arange(m))


@needs_gpu
@pytest.mark.parametrize("m,n,k", [(66560 - 37, 392, 72), (128000, 384, 128), (179200 - 100, 264, 64)])
def test_rows_path_many_row_blocks(native_lib, m, n, k):
    """520 to 1400 row blocks of one batch (two to six workgroups per CU, in
    waves), ragged rows and columns, against the oracle on sampled rows."""
    from welder_typical_chain_amd import _lib
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    pl = _lib.plan(1, m, n, k, 1, 1, _lib.PATH_ROWS, None, cu)
    assert pl["grid"] == -(-m // 128), pl
    cfg = ChainConfig("rows-many", 1, m, n, k, "f16", "f16", "normal", 0.4, logit_scale=0.7)
    _announce(f"rows path, {m}x{n}x{k}")
    inp = O.make_inputs(cfg, seed=13)
    out = run_chain(inp, "f16", "f16", path="rows")
    rows = np.unique(np.concatenate([sample_rows(m, 12, seed=k), np.arange(0, m, 2431), [m - 1]]))
    _check(cfg, inp, out, rows)


@needs_gpu
def test_rows_path_batched_matches_exchange(native_lib):
    cfg = ChainConfig("rows-b", 3, 256, 512, 64, "f16", "f16", "normal", 0.5, logit_scale=0.9)
    _announce("rows path, batch 3 256x512x64, against the oracle and the exchange path")
    inp = O.make_inputs(cfg, seed=9)
    rows = run_chain(inp, "f16", "f16", path="rows", batched=True)
    _check(cfg, inp, rows, np.arange(256), batches=(0, 1, 2))
    exch = run_chain(inp, "f16", "f16", path="exchange", batched=True)
    assert float((rows.float() - exch.float()).abs().max()) < 2e-3


@needs_gpu
def test_c4_wide_rows_bf16(native_lib):
    cfg = CONFIGS["C4"]
    _announce("C4 bf16 1024x32768x4096 split-N")
    inp = O.make_inputs(cfg, seed=0)
    out = run_chain(inp, cfg.in_dtype, cfg.out_dtype)
    _check(cfg, inp, out, sample_rows(cfg.m, 4))


@needs_gpu
def test_c5_fp8(native_lib):
    cfg = CONFIGS["C5"]
    _announce("C5 fp8 8192x8192x4096")
    inp = O.make_inputs(cfg, seed=0)
    out = run_chain(inp, cfg.in_dtype, cfg.out_dtype)
    _check(cfg, inp, out, sample_rows(cfg.m, 6))


@needs_gpu
def test_edge_k0_uniform(native_lib):
    from welder_typical_chain_amd.chain import matmul_softmax
    _announce("K=0 gives uniform rows; M=0 is a no-op")
    a = torch.empty((130, 0), dtype=torch.float16, device="cuda")
    b = torch.empty((0, 136), dtype=torch.float16, device="cuda")
    for path in ("exchange", "split", "unfused"):
        out = matmul_softmax(a, b, path=path)
        torch.cuda.synchronize()
        assert torch.allclose(out.float(), torch.full_like(out.float(), 1.0 / 136), rtol=1e-3, atol=0)
    empty = matmul_softmax(torch.empty((0, 16), dtype=torch.float16, device="cuda"),
                           torch.empty((16, 64), dtype=torch.float16, device="cuda"))
    assert empty.shape == (0, 64)


@needs_gpu
def test_negative_scale_and_shift_invariance(native_lib):
    _announce("negative logit scale; row shift invariance")
    cfg = ChainConfig("neg", 1, 128, 256, 64, "f16", "f32", "normal", 0.5, logit_scale=-0.7)
    inp = O.make_inputs(cfg, seed=11)
    out = run_chain(inp, "f16", "f32")
    _check(cfg, inp, out, np.arange(128))


@needs_gpu
@pytest.mark.parametrize("path,in_dtype,out_dtype,batch,m,n,k", [
    ("exchange", "f16", "f16", 1, 200, 264, 72),
    ("exchange", "bf16", "f32", 3, 130, 136, 64),
    ("split", "f16", "bf16", 1, 200, 1000, 72),
    ("split", "fp8", "f16", 64, 200, 1000, 80),   # 256-row tiles
    ("rows", "f16", "f16", 2, 300, 264, 120),
    ("rows", "bf16", "f32", 1, 64, 4104, 8),
    ("unfused", "f16", "f32", 1, 200, 264, 72),
])
def test_negative_scale_every_path(native_lib, path, in_dtype, out_dtype, batch, m, n, k):
    """A negative logit scale turns each kernel's running row max into a
    min of the accumulators (its own code in every path); ragged M, N, K."""
    cfg = ChainConfig("negscale", batch, m, n, k, in_dtype, out_dtype, "normal", 0.5,
                      logit_scale=-0.9)
    _announce(f"negative scale, {path} {in_dtype}->{out_dtype} {batch}x{m}x{n}x{k}")
    inp = O.make_inputs(cfg, seed=23)
    out = run_chain(inp, in_dtype, out_dtype, path=path, batched=batch > 1)
    batches = (0, batch - 1) if batch > 1 else (0,)
    _check(cfg, inp, out, sample_rows(m, 24), batches=batches, path=path)


@needs_gpu
def test_exchange_repeated_launches_and_workspace_reuse(native_lib):
    """40 exchange launches with changing inputs on one workspace (stale row
    statistics or counters would show as wrong rows), then the same workspace
    reused for a smaller shape and back (the counter region must survive)."""
    import math
    from welder_typical_chain_amd.chain import (matmul_softmax, new_workspace, read_diagnostics,
                                                workspace_size)
    _announce("exchange: 40 launches with changing inputs + workspace reuse across shapes")
    dev = torch.device("cuda")
    m = n = 2048
    k = 1024
    ws = new_workspace(workspace_size(1, m, n, k, 1, 1) + (1 << 20), dev)
    out = torch.empty((m, n), dtype=torch.float16, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    worst = 0.0
    for it in range(40):
        a = (torch.randn((m, k), generator=g, device=dev) * (0.5 + it / 20) / math.sqrt(k)).half()
        b = (torch.randn((k, n), generator=g, device=dev) / math.sqrt(k)).half()
        matmul_softmax(a, b, out=out, path="exchange", workspace=ws)
        ref = torch.softmax(a.float() @ b.float(), dim=-1)
        worst = max(worst, float(((out.float() - ref).abs() / ref).max()))
        if it in (10, 20):  # a different shape on the same workspace, all paths
            for path in ("exchange", "split", "unfused"):
                small = matmul_softmax(a[:200, :64].contiguous(), b[:64, :264].contiguous(),
                                       path=path, workspace=ws)
                sref = torch.softmax(a[:200, :64].float() @ b[:64, :264].float(), dim=-1)
                assert float((small.float() - sref).abs().max()) < 2e-3
    torch.cuda.synchronize()
    flags, longest, timeouts = read_diagnostics(ws)
    print(f"[gpu-case] worst rel err {worst:.3e}; longest wait {longest / 100:.1f} us; timeouts {timeouts}")
    assert worst < 2e-3 and flags == 0 and timeouts == 0


@needs_gpu
@pytest.mark.parametrize("path,shape,in_dt", [("exchange", (1, 1024, 2048, 256), torch.float16),
                                              ("split", (1, 512, 4096, 256), torch.bfloat16),
                                              ("rows", (4, 512, 1024, 128), torch.float16),
                                              ("unfused", (1, 256, 512, 128), torch.float16)])
def test_graph_replay_matches_eager(native_lib, path, shape, in_dt):
    """Calls captured in a HIP graph (torch.cuda.graph) and replayed several
    times, with the program's own eager work and synchronisations between the
    replays, give the eager call's output bit for bit on every replay: the
    launches keep no per-launch host state and record no memset."""
    from welder_typical_chain_amd.chain import matmul_softmax, new_workspace, workspace_size
    batch, m, n, k = shape
    _announce(f"graph replay path={path} batch={batch} {m}x{n}x{k} {in_dt}")
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    bs = (batch,) if batch > 1 else ()
    a = (torch.randn((*bs, m, k), generator=g, device=dev) / k ** 0.5).to(in_dt)
    b = (torch.randn((*bs, k, n), generator=g, device=dev)).to(in_dt)
    code = {torch.float16: 1, torch.bfloat16: 2}[in_dt]
    ws = new_workspace(workspace_size(batch, m, n, k, code, 1, path), dev)
    out = torch.empty((*bs, m, n), dtype=torch.float16, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):  # eager warm-up (library initialisation happens outside capture)
            matmul_softmax(a, b, out=out, path=path, workspace=ws)
    torch.cuda.synchronize()
    ref = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        matmul_softmax(a, b, out=out, path=path, workspace=ws)
        matmul_softmax(a, b, out=out, path=path, workspace=ws)
    torch.cuda.synchronize()
    for rep in range(4):
        out.zero_()
        junk = (a.float() * 2.0).sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}: max diff {(out.float() - ref.float()).abs().max().item()}"
        del junk


@needs_gpu
def test_concurrent_host_threads_on_streams(native_lib):
    """Four host threads, each with its own stream and workspace, call the
    launcher concurrently (the C-ABI call releases the GIL, so the calls
    meet in the library's launch code) on the split, row-block and unfused
    paths; every result must match the torch fp32 reference of its inputs."""
    import threading
    from welder_typical_chain_amd.chain import matmul_softmax, new_workspace, workspace_size
    _announce("4 host threads x 12 calls, own streams and workspaces (split/rows/unfused)")
    dev = torch.device("cuda")
    jobs = [("split", 640, 1000, 256), ("rows", 512, 1024, 128), ("unfused", 300, 520, 64),
            ("split", 256, 4096, 128)]
    errors, worst = [], [0.0] * len(jobs)

    def work(i, path, m, n, k):
        try:
            stream = torch.cuda.Stream(device=dev)
            g = torch.Generator(device=dev)
            g.manual_seed(100 + i)
            with torch.cuda.stream(stream):
                ws = new_workspace(workspace_size(1, m, n, k, 1, 1, path), dev)
                for it in range(12):
                    a = (torch.randn((m, k), generator=g, device=dev) / k ** 0.5).half()
                    b = (torch.randn((k, n), generator=g, device=dev) * (1 + it / 6)).half()
                    out = matmul_softmax(a, b, out_dtype=torch.float16, path=path, workspace=ws)
                    ref = torch.softmax(a.float() @ b.float(), dim=-1)
                    d = (out.float() - ref).abs()
                    bad = d > 2e-3 + 1e-2 * ref
                    worst[i] = max(worst[i], float(d.max()))
                    if bool(bad.any()):
                        errors.append(f"thread {i} ({path}) call {it}: max abs {float(d.max()):.3e}")
                        return
            stream.synchronize()
        except Exception as e:  # reported below, on the main thread
            errors.append(f"thread {i} ({path}): {e!r}")

    threads = [threading.Thread(target=work, args=(i, *j)) for i, j in enumerate(jobs)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    torch.cuda.synchronize()
    print(f"[gpu-case] worst abs err per thread {['%.2e' % w for w in worst]}")
    assert not errors, errors
