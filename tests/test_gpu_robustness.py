"""GPU tests of the launcher's failure reporting and default workspaces.

* A timed-out exchange wait reaches the caller: the wait limit is set to a
  few ticks from the host, so the first tiles of every row block give up
  (every kernel still exits normally: all waits are bounded), and the error
  must come back as WTC_ERR_TIMEOUT from wtc_check_status and from the next
  call on the same stream, once; a call on another stream is not affected.
* wtc_release_stream frees a stream's default workspace.
* Default workspaces: one per stream, grow-only; none is allocated while the
  stream is being captured; a graph captured with the default workspace still
  replays correctly after an eager call of a larger shape grew it.
* Calls from several host threads at once, each on its own stream, give the
  one-thread results.
"""
from __future__ import annotations

import math

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

needs_gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="no GPU")


# K of the timeout tests.  A wait runs out only when a tile's first poll
# misses an entry, i.e. when the tiles of a row block publish further apart
# than a tile takes to publish its own; that spread grows with the K loop.
# Measured on MI355X at M = N = 2048 with a 2-tick limit: K = 256 timed out
# in 0 of 30 calls on one box, K = 1024 in 22 of 30, K = 4096 in 30 of 30
# (hundreds of timed-out waits per call).
K_TIMEOUT = 4096


def _announce(msg: str) -> None:
    print(f"\n[gpu-case] {msg}", flush=True)


def _inputs(m, n, k, seed, dev="cuda"):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = (torch.randn((m, k), generator=g, device=dev) / math.sqrt(k)).half()
    b = torch.randn((k, n), generator=g, device=dev).half()
    return a, b


@needs_gpu
def test_exchange_timeout_is_reported(native_lib):
    from welder_typical_chain_amd import _lib
    from welder_typical_chain_amd.chain import (check_status, matmul_softmax, new_workspace,
                                                read_diagnostics, set_exchange_wait_limit,
                                                workspace_size)
    _announce("exchange wait limit of 2 ticks: timeouts reported, then a clean call")
    m = n = 2048
    k = K_TIMEOUT
    a, b = _inputs(m, n, k, 3)
    ws = new_workspace(workspace_size(1, m, n, k, 1, 1, "exchange"))
    ref = torch.softmax(a.float() @ b.float(), dim=-1)
    try:
        set_exchange_wait_limit(2)  # 20 ns: tiles that finish first give up
        reported = False
        for _ in range(8):
            matmul_softmax(a, b, path="exchange", workspace=ws)
            try:
                check_status()
            except _lib.WtcError as e:
                assert e.code == _lib.WTC_ERR_TIMEOUT, e
                reported = True
                break
        flags, _, timeouts = read_diagnostics(ws)
        print(f"[gpu-case] reported {reported}; workspace flags {flags} timeouts {timeouts}")
        assert reported and flags & 1 and timeouts > 0
        # reported once: the status is clean now
        check_status()
        # a timeout left in the mailbox is reported by the next call, which does nothing else.
        # Whether a call times out at this limit depends on the order the tiles start in, so
        # calls are made until one has (its workspace counts the timed-out waits).
        timed_out = False
        for _ in range(8):
            matmul_softmax(a, b, path="exchange", workspace=ws)
            torch.cuda.synchronize()
            if read_diagnostics(ws)[2] > 0:
                timed_out = True
                break
        assert timed_out
        with pytest.raises(_lib.WtcError) as ei:
            matmul_softmax(a, b, path="exchange", workspace=ws)
        assert ei.value.code == _lib.WTC_ERR_TIMEOUT
    finally:
        set_exchange_wait_limit(0)
    read_diagnostics(ws)  # clear the workspace's words
    out = matmul_softmax(a, b, path="exchange", workspace=ws, check=True)
    err = float((out.float() - ref).abs().max())
    flags, longest, timeouts = read_diagnostics(ws)
    print(f"[gpu-case] clean call: max abs err {err:.2e}, longest wait {longest / 100:.1f} us")
    assert err < 2e-3 and flags == 0 and timeouts == 0


@needs_gpu
def test_timeout_is_reported_to_its_own_stream(native_lib):
    """Stream A's call times out (wait limit of 2 ticks); stream B's next call
    runs and is correct; A's next call reports WTC_ERR_TIMEOUT and does
    nothing else; the call after that on A runs and is correct."""
    from welder_typical_chain_amd import _lib
    from welder_typical_chain_amd.chain import (check_status, matmul_softmax, new_workspace,
                                                read_diagnostics, release_stream,
                                                set_exchange_wait_limit, workspace_size)
    _announce("two streams: A times out at a 2-tick limit, B runs, A's next call reports")
    m = n = 2048
    k = K_TIMEOUT
    a, b = _inputs(m, n, k, 5)
    ref = torch.softmax(a.float() @ b.float(), dim=-1)
    nbytes = workspace_size(1, m, n, k, 1, 1, "exchange")
    ws_a, ws_b = new_workspace(nbytes), new_workspace(nbytes)
    s_a, s_b = torch.cuda.Stream(), torch.cuda.Stream()
    for s in (s_a, s_b):
        s.wait_stream(torch.cuda.current_stream())
    try:
        set_exchange_wait_limit(2)
        timed_out = False
        with torch.cuda.stream(s_a):
            # whether a call times out at this limit depends on the order its tiles start in
            for _ in range(8):
                matmul_softmax(a, b, path="exchange", workspace=ws_a)
                s_a.synchronize()
                if read_diagnostics(ws_a)[2] > 0:
                    timed_out = True
                    break
        assert timed_out
    finally:
        set_exchange_wait_limit(0)
    with torch.cuda.stream(s_b):
        out_b = matmul_softmax(a, b, path="exchange", workspace=ws_b)
        check_status()  # stream B has nothing to report
    s_b.synchronize()
    err_b = float((out_b.float() - ref).abs().max())
    flags_b = read_diagnostics(ws_b)
    print(f"[gpu-case] stream B: max abs err {err_b:.2e}, diagnostics {flags_b}", flush=True)
    assert err_b < 2e-3 and flags_b[0] == 0 and flags_b[2] == 0
    with torch.cuda.stream(s_a):
        stale = torch.full((m, n), 7.0, dtype=torch.float16, device="cuda")
        with pytest.raises(_lib.WtcError) as ei:
            matmul_softmax(a, b, out=stale, path="exchange", workspace=ws_a)
        assert ei.value.code == _lib.WTC_ERR_TIMEOUT
        assert "stream" in str(ei.value)
        check_status()  # reported once
        out_a = matmul_softmax(a, b, path="exchange", workspace=ws_a, check=True)
    s_a.synchronize()
    assert bool((stale == 7.0).all()), "the reporting call wrote its output"
    err_a = float((out_a.float() - ref).abs().max())
    flags_a = read_diagnostics(ws_a)
    print(f"[gpu-case] stream A after the report: max abs err {err_a:.2e}, diagnostics {flags_a}")
    assert err_a < 2e-3 and flags_a[0] == 0 and flags_a[2] == 0
    release_stream(s_a)
    release_stream(s_b)


@needs_gpu
def test_release_stream_frees_its_default_workspace(native_lib):
    from welder_typical_chain_amd.chain import matmul_softmax, release_stream, workspace_size
    m, n, k = 2048, 16384, 64
    need = workspace_size(1, m, n, k, 1, 1, "unfused")
    _announce(f"default workspace of {need >> 20} MiB on a new stream, then released")
    a, b = _inputs(m, n, k, 6)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    with torch.cuda.stream(s):
        out = matmul_softmax(a, b, path="unfused")
    s.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    release_stream(s)
    free2 = torch.cuda.mem_get_info()[0]
    print(f"[gpu-case] free MiB: {free0 >> 20} -> {free1 >> 20} -> {free2 >> 20}", flush=True)
    out_bytes = out.numel() * out.element_size()
    assert free0 - free1 >= need - out_bytes // 2  # the workspace (and perhaps the output)
    assert free2 - free1 >= need * 9 // 10
    # the stream works again afterwards, with a new default workspace
    with torch.cuda.stream(s):
        again = matmul_softmax(a, b, path="unfused")
    s.synchronize()
    assert torch.equal(again, out)
    release_stream(s)


@needs_gpu
def test_default_workspace_not_allocated_during_capture(native_lib):
    from welder_typical_chain_amd import _lib
    from welder_typical_chain_amd.chain import matmul_softmax
    _announce("NULL workspace on a capturing stream without a default workspace is refused")
    a, b = _inputs(256, 512, 64, 5)
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    raised = None
    with torch.cuda.graph(graph, stream=s):
        try:
            matmul_softmax(a, b, path="exchange")
        except _lib.WtcError as e:
            raised = e
    torch.cuda.synchronize()
    assert raised is not None and raised.code == _lib.WTC_ERR_ARG, raised
    assert "captur" in str(raised)


@needs_gpu
def test_graph_with_default_workspace_survives_its_growth(native_lib):
    """A graph captured with the stream's default workspace; then an eager
    call of a larger shape on the same stream grows that workspace; every
    replay of the graph must still match the eager output bit for bit (the
    superseded buffer stays allocated)."""
    from welder_typical_chain_amd.chain import matmul_softmax
    _announce("graph on the default workspace, then the workspace grows, then replays")
    a, b = _inputs(512, 1024, 128, 7)
    big_a, big_b = _inputs(2048, 8192, 128, 8)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out = torch.empty((512, 1024), dtype=torch.float16, device="cuda")
    with torch.cuda.stream(s):
        for _ in range(2):  # creates the stream's default workspace outside the capture
            matmul_softmax(a, b, out=out, path="split")
    torch.cuda.synchronize()
    ref = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        matmul_softmax(a, b, out=out, path="split")
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        big = matmul_softmax(big_a, big_b, path="split")  # needs a larger default workspace
    torch.cuda.synchronize()
    big_ref = torch.softmax(big_a[:64].float() @ big_b.float(), dim=-1)
    assert float((big[:64].float() - big_ref).abs().max()) < 2e-3
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"


@needs_gpu
def test_calls_from_several_host_threads(native_lib):
    """Four host threads, each with its own stream and workspace, call the
    rows, split and unfused paths 8 times each at once (the launcher holds
    its lock only for the shared state, not across these launches); every
    output equals the one-thread result of the same call bit for bit."""
    import threading

    from welder_typical_chain_amd.chain import matmul_softmax, new_workspace, workspace_size

    jobs = [("rows", 2, 300, 520, 64), ("split", 1, 256, 2048, 256), ("unfused", 1, 200, 264, 72)]
    g = torch.Generator(device="cpu").manual_seed(11)
    data = []
    for path, batch, m, n, k in jobs:
        a = (torch.randn(batch, m, k, generator=g) * 0.5).half().cuda()
        b = (torch.randn(batch, k, n, generator=g) * 0.5).half().cuda()
        ref = matmul_softmax(a, b, path=path)
        data.append((path, a, b, ref, workspace_size(batch, m, n, k, 1, 1, path)))
    torch.cuda.synchronize()
    errors = []

    def worker(tid):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                wss = [new_workspace(nb, torch.device("cuda")) for *_, nb in data]
                outs = []
                for _ in range(8):
                    for (path, a, b, _, _), ws in zip(data, wss):
                        outs.append((path, matmul_softmax(a, b, path=path, workspace=ws)))
            stream.synchronize()
            for i, (path, o) in enumerate(outs):
                ref = data[i % len(data)][3]
                if not torch.equal(o, ref):
                    errors.append(f"thread {tid} call {i} ({path}) differs")
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(f"thread {tid}: {e!r}")

    print("\n[gpu-case] 4 host threads x 24 calls (rows, split, unfused)", flush=True)
    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a host thread did not finish"
    assert not errors, errors[:4]
