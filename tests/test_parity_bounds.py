"""CPU checks of the logit error bound the GPU parity tests use
(tests/parity_util.logit_error_bound): it must cover f32 accumulation in k
order under round-to-nearest and under round-toward-zero (every addition off
by less than one ulp), for products of decoded 16-bit and e4m3 inputs (exact
in f32) and of f32 inputs (rounded), and it must not be vacuous."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O

from .parity_util import U32, logit_error_bound


def _f32_accumulate(a_row: np.ndarray, b: np.ndarray, toward_zero: bool, round_products: bool):
    """f32 sum over k of a_k * b_kj in k order; each addition rounded to
    nearest, or toward zero (one ulp down in magnitude when nearest rounded up)."""
    s = np.zeros(b.shape[1], np.float32)
    for kk in range(b.shape[0]):
        p = a_row[kk].astype(np.float64) * b[kk].astype(np.float64)
        if round_products:
            p = p.astype(np.float32).astype(np.float64)
        exact = s.astype(np.float64) + p
        t = exact.astype(np.float32)
        if toward_zero:
            up = np.abs(t.astype(np.float64)) > np.abs(exact)
            t = np.where(up, np.nextafter(t, np.float32(0)), t)
        s = t
    return s.astype(np.float64)


def _inputs(kind: str, k: int, n: int, seed: int):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((4, k)) * 3.0
    b = rng.standard_normal((k, n)) * 2.0
    if kind == "f16":
        return O.from_f16_bits(O.to_f16_bits(a)), O.from_f16_bits(O.to_f16_bits(b))
    if kind == "bf16":
        return O.from_bf16_bits(O.to_bf16_bits(a)), O.from_bf16_bits(O.to_bf16_bits(b))
    if kind == "fp8":
        qa, _ = O.quantize_e4m3_amax(a)
        qb, _ = O.quantize_e4m3_amax(b)
        return O.from_e4m3(qa), O.from_e4m3(qb)
    return a.astype(np.float32), b.astype(np.float32)


@pytest.mark.parametrize("kind", ["f16", "bf16", "fp8", "f32"])
@pytest.mark.parametrize("toward_zero", [False, True])
def test_bound_covers_f32_accumulation(kind, toward_zero):
    k, n = 512, 96
    a, b = _inputs(kind, k, n, seed=7)
    if toward_zero:  # positive terms: the directed-rounding errors add up instead of cancelling
        a, b = np.abs(a), np.abs(b)
    rows = np.arange(4)
    scale = 0.37
    logits, _ = O.chain_rows(a.astype(np.float32), b.astype(np.float32), rows, scale)
    bound = logit_error_bound(a, b, rows, scale, logits, kind)
    worst = 0.0
    for r in rows:
        got = scale * _f32_accumulate(a[r], b, toward_zero, round_products=kind == "f32")
        err = np.abs(got - logits[r])
        assert (err <= bound[r]).all(), (kind, toward_zero, float((err / bound[r]).max()))
        worst = max(worst, float((err / bound[r]).max()))
    # with positive terms, directed rounding of 16-bit products (whose low
    # bits fall below the partial sums' ulp at almost every addition) drifts
    # to a sizeable share of the bound: it is not vacuous.  e4m3 products
    # carry few bits, so most of their additions are exact.
    if toward_zero and kind in ("f16", "bf16"):
        assert worst > 0.1, worst
    print(f"{kind} toward_zero={toward_zero}: worst error / bound {worst:.3f}")


def test_bound_scales_with_the_accumulation():
    """Twice the scale doubles the accumulation term; a zero row has only
    the rounding term of its (zero) logits."""
    a, b = _inputs("f16", 256, 64, seed=3)
    rows = np.arange(2)
    l1, _ = O.chain_rows(a.astype(np.float32), b.astype(np.float32), rows, 1.0)
    l2, _ = O.chain_rows(a.astype(np.float32), b.astype(np.float32), rows, 2.0)
    e1 = logit_error_bound(a, b, rows, 1.0, l1, "f16") - 4 * U32 * np.abs(l1)
    e2 = logit_error_bound(a, b, rows, 2.0, l2, "f16") - 4 * U32 * np.abs(l2)
    np.testing.assert_allclose(e2, 2 * e1, rtol=1e-12)
    z = np.zeros_like(a)
    lz, _ = O.chain_rows(z.astype(np.float32), b.astype(np.float32), rows, 1.0)
    assert (logit_error_bound(z, b, rows, 1.0, lz, "f16") == 0).all()
