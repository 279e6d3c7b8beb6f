"""The allocation-free entry point wtc_matmul_softmax_noalloc, called through
the C-ABI, against wtc_matmul_softmax with a caller workspace: the same
kernels run, so the outputs must be identical bit for bit, on two calls in a
row (the second smaller, reusing the scratch array), on every path; a
problem whose workspace exceeds the array is refused; a captured call
replays correctly, also when it is the first call of the entry point in a
process (after the documented set-up call, wtc_check_status).
"""
from __future__ import annotations

import math

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

needs_gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="no GPU")

SHAPES = {  # (m, n, k) of the first call, then a smaller second call
    "exchange": [(2048, 2048, 512), (256, 384, 64)],
    "split": [(1024, 4096, 256), (200, 1000, 72)],
    "rows": [(512, 2048, 128), (64, 264, 64)],
    "unfused": [(256, 512, 64), (128, 136, 32)],
    "auto": [(2048, 2048, 1024), (300, 520, 96)],
}


def _announce(msg: str) -> None:
    print(f"\n[gpu-case] {msg}", flush=True)


def _inputs(m, n, k, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    a = (torch.randn((m, k), generator=g, device="cuda") / math.sqrt(max(k, 1))).half()
    b = torch.randn((k, n), generator=g, device="cuda").half()
    return a, b


def _noalloc(lib, a, b, out, m, n, k, path, stream):
    from welder_typical_chain_amd import _lib
    return lib.wtc_matmul_softmax_noalloc(a.data_ptr(), b.data_ptr(), out.data_ptr(), 1, m, n, k,
                                          _lib.DTYPE_F16, _lib.DTYPE_F16, 1.0, 1.0, 1.0,
                                          _lib.PATHS[path], stream)


@needs_gpu
@pytest.mark.parametrize("path", list(SHAPES))
def test_noalloc_matches_workspace_entry_point(native_lib, path):
    from welder_typical_chain_amd import _lib
    from welder_typical_chain_amd.chain import matmul_softmax, new_workspace, workspace_size
    lib = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    for i, (m, n, k) in enumerate(SHAPES[path]):
        _announce(f"noalloc {path} call {i + 1}: {m}x{n}x{k} f16")
        a, b = _inputs(m, n, k, 40 + i)
        ws = new_workspace(workspace_size(1, m, n, k, 1, 1, path))
        ref = matmul_softmax(a, b, out_dtype=torch.float16, path=path, workspace=ws)
        out = torch.full((m, n), float("nan"), dtype=torch.float16, device="cuda")
        rc = _noalloc(lib, a, b, out, m, n, k, path, stream)
        assert rc == 0, lib.wtc_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"max diff {(out.float() - ref.float()).abs().max().item()}"
        # and to the fp32 reference of the same inputs (north-star gate)
        exp = torch.softmax(a.float() @ b.float(), dim=-1)
        d = (out.float() - exp).abs()
        assert bool((d <= 2e-3 + 1e-2 * exp).all())
    import ctypes
    words = (ctypes.c_uint32 * 3)()
    assert lib.wtc_read_error_flags(None, words, 1) == 0
    assert words[0] == 0 and words[2] == 0, list(words)


@needs_gpu
def test_noalloc_refuses_oversized_problem(native_lib):
    from welder_typical_chain_amd import _lib
    lib = _lib.lib()
    m, n, k = 8192, 32768, 16
    need = lib.wtc_matmul_softmax_workspace_size(1, m, n, k, 1, 1, _lib.PATH_SPLIT)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    _announce(f"noalloc split {m}x{n}x{k}: workspace {need} bytes > scratch, refused")
    a, b = _inputs(m, n, k, 3)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    rc = _noalloc(lib, a, b, out, m, n, k, "split", torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.WTC_ERR_WORKSPACE
    assert b"allocation-free" in lib.wtc_last_error()


@needs_gpu
def test_noalloc_in_a_captured_graph(native_lib):
    """A noalloc call captured into a graph and replayed with eager work and
    synchronisations between replays matches the eager call bit for bit."""
    from welder_typical_chain_amd import _lib
    _announce("noalloc exchange call captured in a graph, 4 replays")
    lib = _lib.lib()
    m, n, k = 1024, 2048, 256
    a, b = _inputs(m, n, k, 9)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        assert _noalloc(lib, a, b, out, m, n, k, "exchange", s.cuda_stream) == 0
    torch.cuda.synchronize()
    ref = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        assert _noalloc(lib, a, b, out, m, n, k, "exchange", s.cuda_stream) == 0
    torch.cuda.synchronize()
    for rep in range(4):
        out.zero_()
        junk = (a.float() * 3.0).sum()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"
        del junk


_FIRST_CALL_CAPTURED = r"""
import ctypes, sys
import torch
from welder_typical_chain_amd import _lib
lib = _lib.lib()
m, n, k = 1024, 2048, 256
g = torch.Generator(device="cuda")
g.manual_seed(21)
a = (torch.randn((m, k), generator=g, device="cuda") / 16.0).half()
b = torch.randn((k, n), generator=g, device="cuda").half()
out = torch.zeros((m, n), dtype=torch.float16, device="cuda")
ref = torch.zeros_like(out)
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
torch.cuda.synchronize()
def call(o):
    return lib.wtc_matmul_softmax_noalloc(a.data_ptr(), b.data_ptr(), o.data_ptr(), 1, m, n, k,
                                          _lib.DTYPE_F16, _lib.DTYPE_F16, 1.0, 1.0, 1.0,
                                          _lib.PATH_EXCHANGE, s.cuda_stream)
# the library's first call in this process: the device's set-up
assert lib.wtc_check_status(s.cuda_stream) == 0, lib.wtc_last_error()
print("[child] set-up done; capturing the first noalloc call", flush=True)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=s):
    rc = call(out)
assert rc == 0, lib.wtc_last_error()
torch.cuda.synchronize()
with torch.cuda.stream(s):
    assert call(ref) == 0, lib.wtc_last_error()
torch.cuda.synchronize()
exp = torch.softmax(a.float() @ b.float(), dim=-1)
assert float((ref.float() - exp).abs().max()) < 2e-3
for rep in range(3):
    out.zero_()
    junk = (a.float() * 3.0).sum()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"replay {rep}"
    del junk
words = (ctypes.c_uint32 * 3)()
assert lib.wtc_read_error_flags(None, words, 1) == 0
assert words[0] == 0 and words[2] == 0, list(words)
assert lib.wtc_check_status(s.cuda_stream) == 0, lib.wtc_last_error()
print("[child] OK", flush=True)
"""


@needs_gpu
def test_noalloc_first_call_captured_after_set_up(native_lib):
    """In a fresh process, wtc_check_status makes the device's set-up and the
    first noalloc call is made under graph capture: its replays match an
    eager noalloc call bit for bit."""
    import os
    import subprocess
    import sys
    _announce("fresh process: wtc_check_status, then the first noalloc call captured")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED], cwd=root, capture_output=True,
                       text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "[child] OK" in r.stdout
