"""PyTorch-facing entry point of the fused chain.

PyTorch supplies device memory and the current HIP stream; every byte of the
chain is computed by the HIP kernels behind ``wtc_matmul_softmax``.
"""
from __future__ import annotations

import torch

from . import _lib

_IN_DTYPES = {
    torch.float32: _lib.DTYPE_F32,
    torch.float16: _lib.DTYPE_F16,
    torch.bfloat16: _lib.DTYPE_BF16,
    torch.float8_e4m3fn: _lib.DTYPE_FP8_E4M3,
}
_OUT_DTYPES = {
    torch.float32: _lib.DTYPE_F32,
    torch.float16: _lib.DTYPE_F16,
    torch.bfloat16: _lib.DTYPE_BF16,
}


def _code_of(t: torch.Tensor) -> int:
    if t.dtype == torch.uint8:  # raw e4m3 bytes
        return _lib.DTYPE_FP8_E4M3
    try:
        return _IN_DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported input dtype {t.dtype}") from None


def workspace_size(batch: int, m: int, n: int, k: int, in_dtype: int, out_dtype: int,
                   path: str = "auto") -> int:
    size = _lib.lib().wtc_matmul_softmax_workspace_size(batch, m, n, k, in_dtype, out_dtype,
                                                        _lib.PATHS[path])
    if size < 0:
        _lib.check(_lib.WTC_ERR_ARG)
    return int(size)


def new_workspace(nbytes: int, device: torch.device | str = "cuda") -> torch.Tensor:
    """A zero-initialised workspace buffer (256-byte aligned by the allocator)."""
    ws = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(ws.device).cuda_stream
    _lib.check(_lib.lib().wtc_workspace_init(ws.data_ptr(), ws.numel(), stream))
    return ws


def matmul_softmax(a: torch.Tensor, b: torch.Tensor, *, out: torch.Tensor | None = None,
                   out_dtype: torch.dtype | None = None, logit_scale: float = 1.0,
                   scale_a: float = 1.0, scale_b: float = 1.0, path: str = "auto",
                   workspace: torch.Tensor | None = None, check: bool = False,
                   tiles=None) -> torch.Tensor:
    """out = softmax_row(logit_scale * scale_a * scale_b * (a @ b)).

    a: [M, K] or [batch, M, K]; b: [K, N] or [batch, K, N]; contiguous CUDA
    tensors of float32 / float16 / bfloat16 / float8_e4m3fn (or uint8 holding
    e4m3 bytes).  Runs on the current stream of a's device.  `tiles`: the five
    best.json tile parameters of the kernel variant to run
    (wtc_matmul_softmax_tiles; None = the variant the cost model picks).
    With check=True
    the stream is synchronised afterwards and a timed-out exchange wait
    raises WtcError (code WTC_ERR_TIMEOUT) instead of being reported by the
    next call.
    """
    if a.dim() not in (2, 3) or b.dim() != a.dim():
        raise ValueError("a and b must both be 2-D or both 3-D")
    if not (a.is_cuda and b.is_cuda):
        raise ValueError("inputs must be on the GPU")
    if not (a.is_contiguous() and b.is_contiguous()):
        raise ValueError("inputs must be contiguous")
    batched = a.dim() == 3
    batch = a.shape[0] if batched else 1
    m, k = a.shape[-2:]
    k2, n = b.shape[-2:]
    if k != k2 or (batched and b.shape[0] != batch):
        raise ValueError(f"shape mismatch: a {tuple(a.shape)} b {tuple(b.shape)}")
    in_code = _code_of(a)
    if _code_of(b) != in_code:
        raise TypeError("a and b must have the same element type")
    if out_dtype is None:
        out_dtype = out.dtype if out is not None else (
            torch.float32 if in_code == _lib.DTYPE_F32 else torch.float16)
    out_code = _OUT_DTYPES[out_dtype]
    shape = (batch, m, n) if batched else (m, n)
    if out is None:
        out = torch.empty(shape, dtype=out_dtype, device=a.device)
    elif tuple(out.shape) != shape or out.dtype != out_dtype or not out.is_contiguous():
        raise ValueError("out has the wrong shape, dtype or layout")
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    stream = torch.cuda.current_stream(a.device).cuda_stream
    head = (a.data_ptr(), b.data_ptr(), out.data_ptr(), batch, m, n, k, in_code, out_code,
            float(logit_scale), float(scale_a), float(scale_b))
    tail = (_lib.PATHS[path], ws_ptr, ws_bytes, stream)
    if tiles is None:
        fn, call = _lib.lib().wtc_matmul_softmax, head + tail
    else:
        import ctypes
        t = _lib.Tiles(*[int(x) for x in tiles])
        fn, call = _lib.lib().wtc_matmul_softmax_tiles, head + (ctypes.byref(t),) + tail
    if a.device.index == torch.cuda.current_device():
        rc = fn(*call)
    else:  # the library launches on the current device
        with torch.cuda.device(a.device):
            rc = fn(*call)
    if rc:
        _lib.check(rc)
    if check:
        check_status(a.device)
    return out


def check_status(device: torch.device | str | None = None) -> None:
    """Synchronise the current stream of `device` and raise WtcError if an
    exchange-path wait of a call on that stream timed out since the last
    report (wtc_check_status)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        _lib.check(_lib.lib().wtc_check_status(stream))


def set_exchange_wait_limit(ticks: int) -> None:
    """Limit of each exchange-path wait in 100 MHz ticks (0 = automatic:
    200 times the cost model's estimate of the call, between 5 ms and 2 s)."""
    _lib.check(_lib.lib().wtc_set_exchange_wait_limit(int(ticks)))


def release_stream(stream: torch.cuda.Stream | None = None) -> None:
    """Free the default workspace and the timeout-mailbox word of `stream`
    (default: the current stream) after synchronising it
    (wtc_release_stream); raises WtcError for a timeout it still held."""
    s = stream if stream is not None else torch.cuda.current_stream()
    with torch.cuda.device(s.device):
        _lib.check(_lib.lib().wtc_release_stream(s.cuda_stream))


def read_error_flags(workspace: torch.Tensor | None = None, clear: bool = True) -> int:
    """Bit 0 set when an exchange-path wait timed out."""
    return read_diagnostics(workspace, clear)[0]


def read_diagnostics(workspace: torch.Tensor | None = None, clear: bool = True):
    """(flags, longest exchange wait in 100 MHz ticks, timed-out waits) of a
    workspace, or of all default workspaces of the current device."""
    import ctypes
    words = (ctypes.c_uint32 * 3)()
    ptr = workspace.data_ptr() if workspace is not None else None
    _lib.check(_lib.lib().wtc_read_error_flags(ptr, words, int(clear)))
    return int(words[0]), int(words[1]), int(words[2])
