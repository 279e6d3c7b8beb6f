"""Shared helpers of the GPU parity tests: upload oracle inputs, run the HIP
chain through the C-ABI, and compare with the float64 oracle.

Tolerances (stated once, used by every GPU parity test):
  * the north-star gate on 16-bit outputs: |d| <= 2e-3 + 1e-2 * |ref| and
    row sums within 1e-3 of 1 (bf16 outputs: within their rounding bound,
    2^-8 + 1e-4, plus 2^-11 on the split path, whose first pass keeps the
    exponentials in f16 before the rescale rounds them to bf16);
  * a tighter relative gate, because outputs are ~1/N: on entries
    >= 1/(8N), |d| <= REL * ref + FLOOR (f16 out: REL 2e-3 = 4 ulp, FLOOR
    1.2e-7 = two steps of the f16 subnormal grid, which 1/(8N) reaches for
    N >= 2048; bf16 out: REL 1.6e-2 = 4 ulp; f32 out: REL 1e-4);
  * f32 outputs: |d| <= 1e-6 + 1e-4 * |ref|;
  * plus, in the relative gate, the error of the logits themselves, bounded
    from the arithmetic (logit_error_bound): a product of two decoded f16,
    bf16 or e4m3 values is exact in f32 (at most 22 significand bits), an
    f32 x f32 product errs by at most u|a b| (u = 2^-24), and each addition
    of the k-ordered f32 accumulation by less than one ulp of its result,
    2u|s_i|, whatever the rounding mode; so |dy_j| <= 2u sum_i |s_i| (+ u
    sum_k |a_k b_kj| for f32 inputs), with the partial sums s_i computed
    exactly from the inputs, plus 4u|y_j| for the scale's and exponent's own
    roundings.  An output p_j = exp(y_j - L) then carries at most
    expm1(|dy_j| + max_i |dy_i|) relative error (L, the log-sum-exp, moves
    by at most the largest |dy_i|);
  * that worst case grows with K like sum_i |s_i| and lets a few percent
    through at large K (C5: 0.07-0.09 logit units, 15-19 % on an output),
    so the gate uses the smaller of it and a statistical bound,
    LAMBDA u sqrt(sum_i s_i^2) (+ the same product and scale terms): with
    rounding errors of at most u|s_i| that do not all lean one way, their
    sum has a standard deviation of about u sqrt(sum_i s_i^2 / 3), so
    LAMBDA = 8 is about 14 of them (C5: about 5e-3 logit units against a
    measured 2.3e-3, about 1 % on an output); and the relative allowance
    this leaves is asserted to stay below LOGIT_REL_CEILING;
  * row argmax agreement wherever the oracle's top two logits differ by more
    than 1e-3 of the row's largest logit and by more than twice its largest
    logit error bound.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

ATOL_NS, RTOL_NS = 2e-3, 1e-2
ROWSUM_TOL = 1e-3
# A bf16 output (8-bit significand) rounds each entry with relative error up
# to u = 2^-8, so its row sum may be off by up to u * sum(p) = 2^-8; the
# north star's 1e-3 is for f16 outputs (u = 2^-11).  The split path first
# stores exp2(y - tile max) in f16 (for bf16 outputs; in the output type
# otherwise) and rescales that in place: one more rounding of 2^-11.  1e-4
# covers the f32 arithmetic before.
BF16_U = 2.0 ** -8
F16_U = 2.0 ** -11
REL = {"f16": 2e-3, "bf16": 1.6e-2, "f32": 1e-4}
FLOOR = {"f16": 1.2e-7, "bf16": 0.0, "f32": 0.0}
U32 = 2.0 ** -24  # unit roundoff of f32 round-to-nearest
LAMBDA = 8.0  # the statistical logit bound, in units of u * sqrt(sum_i s_i^2)
# Largest relative allowance the logit error may add to an output's gate: a
# gate wider than this could hide a systematic error of a few percent (a
# wrong scale, a bad rescale factor).
LOGIT_REL_CEILING = 0.03

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


def logit_error_bound(a: np.ndarray, b: np.ndarray, rows, scale: float, logits: np.ndarray,
                      in_dtype: str, chunk: int = 1 << 20, worst_case: bool = False) -> np.ndarray:
    """Bound on |GPU logit - exact logit| (natural-log units, the units of the
    oracle's logits) for each sampled row and column, from the f32 arithmetic
    described in this module's docstring: the partial sums s_i of the
    k-ordered accumulation are formed exactly (float64 sums of exact
    products).  worst_case: the rigorous bound 2u sum_i |s_i| only;
    otherwise (the gate) the smaller of it and LAMBDA u sqrt(sum_i s_i^2).
    a, b: the decoded inputs of one batch (the oracle's); logits:
    oracle.chain_rows's for the same rows."""
    rows = np.asarray(rows, np.int64)
    ar = np.asarray(a, np.float64)[rows]
    b = np.asarray(b, np.float64)
    k, n = b.shape
    err = np.empty((rows.size, n), np.float64)
    cols = max(1, min(n, chunk // max(1, rows.size)))
    for c0 in range(0, n, cols):
        bc = b[:, c0:c0 + cols]
        s = np.zeros((rows.size, bc.shape[1]))
        sum_abs_s = np.zeros_like(s)
        sum_sq_s = np.zeros_like(s)
        sum_abs_p = np.zeros_like(s)
        sum_sq_p = np.zeros_like(s)
        for kk in range(k):
            prod = ar[:, kk:kk + 1] * bc[kk][None, :]
            s += prod
            sum_abs_s += np.abs(s)
            sum_sq_s += s * s
            if in_dtype == "f32":
                sum_abs_p += np.abs(prod)
                sum_sq_p += prod * prod
        worst = 2.0 * U32 * sum_abs_s + U32 * sum_abs_p
        if worst_case:
            err[:, c0:c0 + cols] = worst
        else:
            stat = LAMBDA * U32 * (np.sqrt(sum_sq_s) + np.sqrt(sum_sq_p))
            err[:, c0:c0 + cols] = np.minimum(worst, stat)
    return abs(scale) * err + 4.0 * U32 * np.abs(logits)


def compare_rows(out_rows: np.ndarray, probs: np.ndarray, logits: np.ndarray, out_dtype: str,
                 label: str = "", in_dtype: str = "f16", logit_err: np.ndarray | None = None) -> dict:
    """Check sampled output rows against the oracle; returns the metrics.
    logit_err: logit_error_bound of the same rows (required)."""
    assert logit_err is not None and logit_err.shape == logits.shape, "logit_error_bound is required"
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
    dmax = logit_err.max(axis=1, keepdims=True)
    rel_logit = np.expm1(logit_err + dmax)
    metrics["max_logit_rel_allowance"] = float(rel_logit.max())
    assert metrics["max_logit_rel_allowance"] <= LOGIT_REL_CEILING, (
        f"{label}: the logit error allowance ({metrics['max_logit_rel_allowance']:.2e}) exceeds "
        f"{LOGIT_REL_CEILING}: the gate would hide errors of that size")
    allow = (REL[out_dtype] + rel_logit) * probs + FLOOR[out_dtype]
    over = d[big] > allow[big]
    assert not over.any(), (
        f"{label}: relative error {metrics['max_rel_big']:.3e} > {REL[out_dtype]:.1e} + logit error "
        f"bound (up to {metrics['max_logit_rel_allowance']:.2e})")
    # argmax agreement where the top-2 logit gap is resolvable
    srt = np.sort(logits, axis=1)
    gap = srt[:, -1] - srt[:, -2]
    scale = np.abs(logits).max(axis=1) + 1e-30
    resolvable = (gap > 1e-3 * scale) & (gap > 2.0 * dmax[:, 0])
    agree = np.argmax(out_rows, axis=1) == np.argmax(logits, axis=1)
    # equal outputs after rounding may tie: accept when the chosen entry equals the max
    tie_ok = out_rows[np.arange(len(out_rows)), np.argmax(logits, axis=1)] == out_rows.max(axis=1)
    assert (agree | tie_ok | ~resolvable).all(), f"{label}: row argmax differs"
    metrics["rows"] = int(len(out_rows))
    return metrics


def check_row_sums(out: torch.Tensor, label: str = "", split: bool = False) -> float:
    """Row sums within 1e-3 of 1 (f16 and f32 outputs) or within the bf16
    rounding bound 2^-8 + 1e-4 (+ 2^-11 for the split path's f16
    intermediate)."""
    s = out.float().sum(dim=-1)
    dev = float((s - 1.0).abs().max())
    tol = BF16_U + (F16_U if split else 0.0) + 1e-4 if out.dtype == torch.bfloat16 else ROWSUM_TOL
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
