"""CPU checks of the row-sum bounds the GPU parity tests use for bf16 outputs
(tests/parity_util.py): rounding exact softmax rows to bf16 once (exchange,
rows, unfused paths) never moves a row sum by more than 2^-8, bf16's unit
roundoff; the split path, which stores exp2(y - tile max) in f16 and then
rescales it in place into bf16, stays within 2^-8 + 2^-11, where storing the
intermediate in bf16 (two bf16 roundings) can go past that; and a single
rounding alone can exceed the north star's 1e-3, which is why bf16 outputs
get their own bound."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from .parity_util import BF16_U, F16_U  # noqa: E402


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


def _f16_scaled(x: np.ndarray) -> np.ndarray:
    """The split path's intermediate for bf16 outputs: f16 of x * 2^15 (exact
    scaling), read back divided by 2^15."""
    return (x * 2.0 ** 15).astype(np.float16).astype(np.float64) / 2.0 ** 15


def _split_rows(y: np.ndarray, stage):
    """Split path on rows y: per 128-column tile, e = exp(y - tile max)
    rounded by `stage`, then e * exp(tile max - row max) / row sum rounded to
    bf16."""
    rows, n = y.shape
    tiles = y.reshape(rows, n // 128, 128)
    tmax = tiles.max(axis=2, keepdims=True)
    e = stage(np.exp(tiles - tmax))
    gmax = y.max(axis=1)[:, None, None]
    s = np.exp(tiles - gmax).sum(axis=(1, 2))[:, None, None]
    return _bf16(e * np.exp(tmax - gmax) / s).reshape(rows, n)


@pytest.mark.parametrize("spread", [0.1, 1.0, 3.0, 6.0])
def test_split_path_f16_intermediate_within_bound(spread):
    rng = np.random.default_rng(2)
    y = rng.standard_normal((300, 1024)) * spread
    out = _split_rows(y, _f16_scaled)
    dev = np.abs(out.sum(axis=1) - 1.0)
    assert dev.max() <= BF16_U + F16_U
    exact = np.exp(y - y.max(axis=1, keepdims=True))
    exact /= exact.sum(axis=1, keepdims=True)
    # one bf16 rounding (unit roundoff 2^-8) of a value within 2^-11 of the
    # exact one, wherever the scaled intermediate is an f16 normal (>= 2^-29)
    big = exact >= 2.0 ** -29
    assert np.all(np.abs(out - exact)[big] <= (BF16_U + F16_U) * exact[big])


def test_bf16_intermediate_rounds_twice():
    """What the f16 intermediate avoids: with the exponentials kept in bf16
    the elementwise error reaches past one bf16 rounding plus 2^-11."""
    rng = np.random.default_rng(3)
    y = rng.standard_normal((300, 1024)) * 3.0
    exact = np.exp(y - y.max(axis=1, keepdims=True))
    exact /= exact.sum(axis=1, keepdims=True)
    big = exact >= 1e-6
    rel_f16 = (np.abs(_split_rows(y, _f16_scaled) - exact) / exact)[big].max()
    rel_bf16 = (np.abs(_split_rows(y, _bf16) - exact) / exact)[big].max()
    assert rel_f16 <= BF16_U + F16_U < rel_bf16


def test_one_rounding_can_exceed_the_f16_bound():
    worst = max(np.abs(_bf16(_rows(seed, 1000, 200, 2.5)).sum(axis=1) - 1.0).max()
                for seed in range(4))
    assert worst > 1e-3
