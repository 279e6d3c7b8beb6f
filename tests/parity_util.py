"""Shared helpers of the GPU parity tests: upload oracle inputs, run the HIP
chain through the C-ABI, and compare with the float64 oracle.

Tolerances (stated once, used by every GPU parity test):
  * the north-star gate on 16-bit outputs: |d| <= 2e-3 + 1e-2 * |ref| and
    row sums within 1e-3 of 1 (bf16 outputs: within their rounding bound,
    2^-8 per rounding + 1e-4, two roundings on the split path);
  * a tighter relative gate, because outputs are ~1/N: on entries
    >= 1/(8N), |d| <= REL * ref + FLOOR (f16 out: REL 2e-3 = 4 ulp, FLOOR
    1.2e-7 = two steps of the f16 subnormal grid, which 1/(8N) reaches for
    N >= 2048; bf16 out: REL 1.6e-2 = 4 ulp; f32 out: REL 1e-4);
  * f32 outputs: |d| <= 1e-6 + 1e-4 * |ref|;
  * plus, in the relative gate, the error of the logits themselves: an output
    p_j = exp(y_j - max) carries the error of y_j - max, bounded here by
    LOGIT_REL * max|y| of the row.  LOGIT_REL is 1e-6 for f32-accumulated
    16-bit and f32 products; for fp8 inputs it is 2e-5, which covers the
    e4m3 MFMA's accumulation measured on MI355X (logit-difference error
    ~8e-6 relative on C5's logits of magnitude ~270);
  * row argmax agreement wherever the oracle's top two logits differ by more
    than the logit error bound.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

ATOL_NS, RTOL_NS = 2e-3, 1e-2
ROWSUM_TOL = 1e-3
# A bf16 output (8-bit significand) rounds each entry with relative error up
# to u = 2^-8, so its row sum may be off by up to u * sum(p) = 2^-8 per
# rounding; the north star's 1e-3 is for f16 outputs (u = 2^-11).  The split path rounds
# twice (it stores exp2(y - tile max) in the output type and rescales that in
# place), the other paths once.  1e-4 covers the f32 arithmetic before.
BF16_U = 2.0 ** -8
REL = {"f16": 2e-3, "bf16": 1.6e-2, "f32": 1e-4}
FLOOR = {"f16": 1.2e-7, "bf16": 0.0, "f32": 0.0}
LOGIT_REL = {"fp8": 2e-5}

_TORCH_OUT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def to_device(raw: np.ndarray, in_dtype: str, device="cuda") -> torch.Tensor:
    if in_dtype == "f32":
        return torch.from_numpy(np.ascontiguousarray(raw)).to(device)
    if in_dtype == "f16":
        return torch.from_numpy(np.ascontiguousarray(raw).view(np.float16)).to(device)
    if in_dtype == "bf16":
        return torch.from_numpy(np.ascontiguousarray(raw).view(np.int16)).to(device).view(torch.bfloat16)
    if in_dtype == "fp8":
        return torch.from_numpy(np.ascontiguousarray(raw)).to(device).view(torch.float8_e4m3fn)
    raise ValueError(in_dtype)


def run_chain(inp: O.ChainInputs, in_dtype: str, out_dtype: str, path: str = "auto",
              batched: bool | None = None, workspace=None, tiles=None) -> torch.Tensor:
    from welder_typical_chain_amd.chain import matmul_softmax
    a = to_device(inp.a_raw, in_dtype)
    b = to_device(inp.b_raw, in_dtype)
    if batched is None:
        batched = a.shape[0] > 1
    if not batched:
        a, b = a[0], b[0]
    out = matmul_softmax(a, b, out_dtype=_TORCH_OUT[out_dtype], logit_scale=inp.logit_scale,
                         scale_a=inp.scale_a, scale_b=inp.scale_b, path=path,
                         workspace=workspace, tiles=tiles)
    torch.cuda.synchronize()
    return out


def compare_rows(out_rows: np.ndarray, probs: np.ndarray, logits: np.ndarray, out_dtype: str,
                 label: str = "", in_dtype: str = "f16") -> dict:
    """Check sampled output rows against the oracle; returns the metrics."""
    out_rows = np.asarray(out_rows, np.float64)
    n = probs.shape[1]
    assert np.isfinite(out_rows).all(), f"{label}: non-finite outputs"
    d = np.abs(out_rows - probs)
    metrics = {"max_abs": float(d.max())}
    if out_dtype == "f32":
        bad = d > 1e-6 + REL["f32"] * np.abs(probs)
        assert not bad.any(), f"{label}: f32 outputs off, max_abs {d.max():.3e}"
    else:
        bad = d > ATOL_NS + RTOL_NS * np.abs(probs)
        assert not bad.any(), f"{label}: north-star tolerance violated, max_abs {d.max():.3e}"
    big = probs >= 1.0 / (8 * n)
    rel = d[big] / probs[big]
    metrics["max_rel_big"] = float(rel.max()) if rel.size else 0.0
    logit_err = LOGIT_REL.get(in_dtype, 1e-6) * np.abs(logits).max(axis=1, keepdims=True)
    allow = (REL[out_dtype] + np.broadcast_to(logit_err, probs.shape)) * probs + FLOOR[out_dtype]
    over = d[big] > allow[big]
    assert not over.any(), (
        f"{label}: relative error {metrics['max_rel_big']:.3e} > {REL[out_dtype]:.1e}")
    # argmax agreement where the top-2 logit gap is resolvable
    srt = np.sort(logits, axis=1)
    gap = srt[:, -1] - srt[:, -2]
    scale = np.abs(logits).max(axis=1) + 1e-30
    resolvable = gap > 1e-3 * scale
    agree = np.argmax(out_rows, axis=1) == np.argmax(logits, axis=1)
    # equal outputs after rounding may tie: accept when the chosen entry equals the max
    tie_ok = out_rows[np.arange(len(out_rows)), np.argmax(logits, axis=1)] == out_rows.max(axis=1)
    assert (agree | tie_ok | ~resolvable).all(), f"{label}: row argmax differs"
    metrics["rows"] = int(len(out_rows))
    return metrics


def check_row_sums(out: torch.Tensor, label: str = "", roundings: int = 1) -> float:
    """Row sums within 1e-3 of 1 (f16 and f32 outputs) or within the bf16
    rounding bound `roundings` * 2^-8 + 1e-4."""
    s = out.float().sum(dim=-1)
    dev = float((s - 1.0).abs().max())
    tol = roundings * BF16_U + 1e-4 if out.dtype == torch.bfloat16 else ROWSUM_TOL
    assert dev <= tol, f"{label}: row sum off by {dev:.3e} (bound {tol:.2e})"
    assert bool(torch.isfinite(out).all()), f"{label}: non-finite outputs"
    return dev


def sample_rows(m: int, count: int, seed: int = 0) -> np.ndarray:
    """First, last and a few seeded middle rows (the reference verifier picks
    0,1,2,3,7,15,...; verify_matmul_softmax.py:166)."""
    fixed = [r for r in (0, 1, 2, 3, 7, 15, 31, 63, 127, 255, 511, 1023) if r < m]
    rng = np.random.default_rng(seed)
    extra = rng.choice(m, size=min(count, m), replace=False)
    rows = sorted(set(fixed) | set(int(x) for x in extra) | {m - 1})
    return np.asarray(rows, np.int64)
