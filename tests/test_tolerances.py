"""CPU checks of the row-sum bounds the GPU parity tests use for bf16 outputs
(tests/parity_util.py): rounding exact softmax rows to bf16 once (exchange,
rows, unfused paths) or twice (the split path stores exp2(y - tile max) in the
output type, then rescales it in place) never moves a row sum by more than
2^-8, bf16's unit roundoff, per rounding; and a single rounding alone can
exceed the north star's 1e-3, which is why bf16 outputs get their own bound."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from .parity_util import BF16_U  # noqa: E402


def _rows(seed: int, n: int, rows: int, spread: float) -> np.ndarray:
    rng = np.random.default_rng(seed)
    y = rng.standard_normal((rows, n)) * spread
    e = np.exp(y - y.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).double().numpy()


@pytest.mark.parametrize("spread", [0.1, 1.0, 3.0, 6.0])
def test_one_rounding_within_u(spread):
    p = _rows(1, 1000, 400, spread)
    dev = np.abs(_bf16(p).sum(axis=1) - 1.0)
    assert dev.max() <= BF16_U


@pytest.mark.parametrize("spread", [0.1, 1.0, 3.0, 6.0])
def test_two_roundings_within_2u(spread):
    """Split path: per 128-column tile, e = exp2(y - tile max) rounded, then
    e * exp2(tile max - row max) / row sum rounded again."""
    rng = np.random.default_rng(2)
    n, rows = 1024, 300
    y = rng.standard_normal((rows, n)) * spread
    tiles = y.reshape(rows, n // 128, 128)
    tmax = tiles.max(axis=2, keepdims=True)
    e = _bf16(np.exp(tiles - tmax))
    gmax = y.max(axis=1)[:, None, None]
    s = np.exp(tiles - gmax).sum(axis=(1, 2))[:, None, None]
    out = _bf16(e * np.exp(tmax - gmax) / s).reshape(rows, n)
    dev = np.abs(out.sum(axis=1) - 1.0)
    assert dev.max() <= 2 * BF16_U
    exact = np.exp(y - y.max(axis=1, keepdims=True))
    exact /= exact.sum(axis=1, keepdims=True)
    assert np.abs(out - exact).max() <= 2.01 * BF16_U * exact.max()


def test_one_rounding_can_exceed_the_f16_bound():
    worst = max(np.abs(_bf16(_rows(seed, 1000, 200, 2.5)).sum(axis=1) - 1.0).max()
                for seed in range(4))
    assert worst > 1e-3
