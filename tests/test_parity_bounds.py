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
    bound = logit_error_bound(a, b, rows, scale, logits, kind, worst_case=True)
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
    e1 = logit_error_bound(a, b, rows, 1.0, l1, "f16", worst_case=True) - 4 * U32 * np.abs(l1)
    e2 = logit_error_bound(a, b, rows, 2.0, l2, "f16", worst_case=True) - 4 * U32 * np.abs(l2)
    np.testing.assert_allclose(e2, 2 * e1, rtol=1e-12)
    z = np.zeros_like(a)
    lz, _ = O.chain_rows(z.astype(np.float32), b.astype(np.float32), rows, 1.0)
    assert (logit_error_bound(z, b, rows, 1.0, lz, "f16") == 0).all()


@pytest.mark.parametrize("kind", ["f16", "fp8", "f32"])
def test_gate_covers_round_to_nearest_accumulation(kind):
    """The gate (the smaller of the worst case and LAMBDA u sqrt(sum s_i^2))
    covers f32 round-to-nearest accumulation in k order with room to spare."""
    k, n = 2048, 64
    a, b = _inputs(kind, k, n, seed=5)
    rows = np.arange(4)
    logits, _ = O.chain_rows(a.astype(np.float32), b.astype(np.float32), rows, 1.0)
    gate = logit_error_bound(a, b, rows, 1.0, logits, kind)
    assert (gate <= logit_error_bound(a, b, rows, 1.0, logits, kind, worst_case=True)).all()
    for r in rows:
        got = _f32_accumulate(a[r], b, False, round_products=kind == "f32")
        err = np.abs(got - logits[r])
        assert (err <= 0.5 * gate[r]).all(), (kind, float((err / gate[r]).max()))


def test_gate_on_c5_is_tight_and_catches_a_scale_error():
    """On C5's inputs (fp8, K = 4096) the worst-case allowance would let 15-19 %
    through on the largest outputs; the gate allows about 1 %, stays below the
    ceiling, and rejects outputs computed with a logit scale 2 % off (a
    mistake planted in the oracle's softmax here, on the CPU)."""
    from welder_typical_chain_amd.configs import CONFIGS
    from .parity_util import LOGIT_REL_CEILING, compare_rows
    cfg = CONFIGS["C5"]
    inp = O.make_inputs(cfg, seed=0, m=64)
    rows = np.array([0, 37])
    logits, probs = O.chain_rows(inp.a[0], inp.b[0], rows, inp.scale)
    worst = logit_error_bound(inp.a[0], inp.b[0], rows, inp.scale, logits, "fp8", worst_case=True)
    gate = logit_error_bound(inp.a[0], inp.b[0], rows, inp.scale, logits, "fp8")
    rel_worst = float(np.expm1(worst + worst.max(axis=1, keepdims=True)).max())
    rel_gate = float(np.expm1(gate + gate.max(axis=1, keepdims=True)).max())
    assert rel_worst > 0.1 > LOGIT_REL_CEILING > 0.02 > rel_gate, (rel_worst, rel_gate)
    # the oracle's own outputs pass
    compare_rows(probs, probs, logits, "f16", "c5-exact", "fp8", gate)
    # a 2 % scale error does not
    y = logits * 1.02
    bad = np.exp(y - y.max(axis=1, keepdims=True))
    bad /= bad.sum(axis=1, keepdims=True)
    with pytest.raises(AssertionError):
        compare_rows(bad, probs, logits, "f16", "c5-scale", "fp8", gate)
