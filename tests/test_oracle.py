"""Pins the CPU oracle (oracle/wtc_oracle.c) before it is trusted as the
checker of the HIP kernels.  CPU only.

Each check is chosen so that a plausible mistake in the oracle fails it:
  * generators against the reference's closed forms, evaluated here
    independently in pure Python (WelderProfilerRuntime.h:136-149,
    verify_matmul_softmax.py:43-63), bit for bit;
  * f16 / bf16 / e4m3 converters against numpy float16 and torch bfloat16 /
    float8_e4m3fn, over every f16 bit pattern and dense random samples;
  * the chain against numpy float64 brute force, and against closed forms
    (all-equal rows -> 1/N, one dominant logit -> one-hot, K = 1, shift
    invariance, scale);
  * the f16-accumulate variant against a numpy float16 loop;
  * the f32 loops baseline against the float64 chain;
  * the committed golden fixtures (tests/golden/).
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _xorshift32(s: int) -> int:
    s &= 0xFFFFFFFF
    s ^= (s << 13) & 0xFFFFFFFF
    s ^= s >> 17
    s ^= (s << 5) & 0xFFFFFFFF
    return s & 0xFFFFFFFF


def _f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


# ----------------------------------------------------------------- generators
def test_xorshift32_sequence():
    lib = O.lib()
    assert lib.wtc_ref_xorshift32(1) == 270369  # 1 ^ 1<<13 = 8193; ^ 8193>>17 = 8193; ^ 8193<<5
    s_py, s_c = 1, 1
    for _ in range(1000):
        s_py = _xorshift32(s_py)
        s_c = lib.wtc_ref_xorshift32(s_c)
        assert s_py == s_c


def test_random_fill_matches_profiler_closed_form():
    # seed 0 behaves as seed 1; u = f32(rng) * 2^-32; value = u*2 - 1 in f32
    for seed in (0, 1, 7, 123456789):
        got = O.fill_random(257, seed)
        s = 1 if seed == 0 else seed
        want = []
        for _ in range(257):
            s = _xorshift32(s)
            u = np.float32(s) * np.float32(1.0 / 4294967296.0)
            want.append(np.float32(u * np.float32(2.0) - np.float32(1.0)))
        np.testing.assert_array_equal(got, np.array(want, np.float32))
    assert np.all(O.fill_random(4096, 3) >= -1.0) and np.all(O.fill_random(4096, 3) <= 1.0)


def test_linear_fill_closed_form():
    got = O.fill_linear(3000)
    idx = np.arange(3000)
    want = (idx % 1024).astype(np.float32) * np.float32(0.001) - np.float32(0.5)
    np.testing.assert_array_equal(got, want)
    assert got[0] == np.float32(-0.5) and got[1024] == np.float32(-0.5)


def test_uniform_fill_reduces_to_random_fill():
    np.testing.assert_array_equal(O.fill_uniform(999, 5, -1.0, 1.0), O.fill_random(999, 5))


def test_normal_fill_moments_and_prefix():
    x = O.fill_normal(1 << 20, 11, 1.0).astype(np.float64)
    assert abs(x.mean()) < 5e-3
    assert abs(x.std() - 1.0) < 5e-3
    assert abs((x ** 3).mean()) < 2e-2          # symmetric
    assert abs((x ** 4).mean() - 3.0) < 5e-2    # gaussian kurtosis
    y = O.fill_normal(8, 11, 2.0)
    np.testing.assert_allclose(y, 2.0 * O.fill_normal(8, 11, 1.0), rtol=1e-6)


# -------------------------------------------------------------------- formats
def test_f16_roundtrip_all_bit_patterns_against_numpy():
    bits = np.arange(1 << 16, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = O.from_f16_bits(bits)
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(got[finite], ref[finite])
    assert np.all(np.isnan(got[np.isnan(ref)]))
    back = O.to_f16_bits(got[finite])
    np.testing.assert_array_equal(back, bits[finite])


def test_f16_rounding_against_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 5, 200000),
        np.float32([65504.0, 65519.0, 65520.0, 1e6, -1e6, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0.0, -0.0]),
        # exact ties between adjacent f16 values
        (np.arange(1, 2000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
    ]).astype(np.float32)
    np.testing.assert_array_equal(O.to_f16_bits(x), x.astype(np.float16).view(np.uint16))


def test_profiler_f16_conversion_differs_only_on_ties():
    # WelderProfilerEval.h:50-100 adds half an ulp and truncates (ties away from zero)
    lib = O.lib()
    x = np.float32(1.0 + 2.0 ** -11)  # exactly between 1.0 and the next f16 value
    assert lib.wtc_ref_f32_to_f16(x) == 0x3C00          # RNE: to even (1.0)
    assert lib.wtc_ref_f32_to_f16_profiler(x) == 0x3C01  # ties away
    y = np.float32(1.3)
    assert lib.wtc_ref_f32_to_f16(y) == lib.wtc_ref_f32_to_f16_profiler(y)


def _f16_ulp(a: np.ndarray) -> np.ndarray:
    """f16 spacing at |a| (float64): 2^(e - 10) in the binade 2^e, 2^-24 below 2^-14."""
    e = np.floor(np.log2(np.maximum(np.abs(a), 2.0 ** -40)))
    return 2.0 ** (np.maximum(e, -14.0) - 10.0)


def _profiler_closed_form(x: np.ndarray) -> np.ndarray:
    """Round to the nearest f16, ties away from zero, overflow to inf (the
    rounding WelderProfilerEval.h:50-100 implements), restated in float64."""
    a = np.abs(x.astype(np.float64))
    ulp = _f16_ulp(a)
    r = np.floor(a / ulp + 0.5) * ulp
    r = np.where(r > 65504.0, np.inf, r)
    return (np.copysign(r, x.astype(np.float64))).astype(np.float16).view(np.uint16)


def test_profiler_f16_conversion_pinned():
    """The profiler's f32 -> f16 over every range: on values that are not
    exact ties it equals IEEE round-to-nearest (numpy), on exact ties it
    rounds away from zero, including ties whose rounding carries into the
    exponent and ties at the subnormal and overflow ends."""
    lib = O.lib()
    conv = np.vectorize(lambda v: lib.wtc_ref_f32_to_f16_profiler(np.float32(v)), otypes=[np.uint16])
    rng = np.random.default_rng(11)
    parts = [
        rng.uniform(2.0 ** -14, 65504.0, 4000),          # normal
        2.0 ** rng.uniform(-14, 16, 4000),                # normal, every binade
        rng.uniform(2.0 ** -25, 2.0 ** -14, 3000),        # subnormal results
        rng.uniform(0.0, 2.0 ** -25, 500),                # below half the smallest subnormal
        rng.uniform(65504.0, 2.0 ** 17, 1000),            # overflow side
    ]
    x = np.concatenate(parts).astype(np.float32)
    x = np.concatenate([x, -x])
    q = np.abs(x.astype(np.float64)) / _f16_ulp(x.astype(np.float64))
    tie = (q - np.floor(q)) == 0.5
    got = conv(x)
    np.testing.assert_array_equal(got[~tie], x[~tie].astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(got[tie], _profiler_closed_form(x[tie]))
    # exact ties: (k + 1/2) ulp in normal binades, at the binade top (k = 2047:
    # the rounding carries into the exponent), in the subnormal range, the
    # smallest subnormal's tie 2^-25, and the overflow tie 65520
    e = rng.integers(-14, 16, 3000)
    k = rng.integers(1024, 2048, 3000)
    ties = [(k + 0.5) * 2.0 ** (e - 10.0), (2047 + 0.5) * 2.0 ** (np.arange(-14, 16) - 10.0),
            (rng.integers(1, 1024, 1000) + 0.5) * 2.0 ** -24, np.array([2.0 ** -25, 65520.0])]
    t = np.concatenate(ties).astype(np.float32)
    t = np.concatenate([t, -t])
    assert ((np.abs(t.astype(np.float64)) / _f16_ulp(t.astype(np.float64))) % 1 == 0.5).all()
    got = conv(t)
    np.testing.assert_array_equal(got, _profiler_closed_form(t))
    # against IEEE these ties differ exactly where RNE rounds down to even
    rne = t.astype(np.float16).view(np.uint16)
    assert (got != rne).any() and (got == rne).any()
    assert lib.wtc_ref_f32_to_f16_profiler(np.float32(2047.5 * 2.0 ** -10)) == 0x4000  # carry to 2.0
    assert lib.wtc_ref_f32_to_f16_profiler(np.float32(65520.0)) == 0x7C00
    assert lib.wtc_ref_f32_to_f16_profiler(np.float32(2.0 ** -25)) == 0x0001
    for v in (np.inf, -np.inf):
        assert lib.wtc_ref_f32_to_f16_profiler(np.float32(v)) == np.float16(v).view(np.uint16)
    assert lib.wtc_ref_f32_to_f16_profiler(np.float32(np.nan)) & 0x7C00 == 0x7C00


def test_bf16_against_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-30, 30, 100000)).astype(np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, 1.0, 3.0e38, -3.0e38])])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.to_bf16_bits(x), want)
    np.testing.assert_array_equal(O.from_bf16_bits(want), torch.from_numpy(want.view(np.int16)).view(
        torch.bfloat16).float().numpy())


def test_e4m3_against_torch():
    torch = pytest.importorskip("torch")
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = O.from_e4m3(codes)
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(got[finite], ref[finite])
    assert np.all(np.isnan(got[~finite]))
    assert ref[finite].max() == 448.0
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.uniform(-448, 448, 200000), rng.standard_normal(50000) * 0.01,
                        np.float32([0.0, 0.001953125, 0.0009765625, 0.00146484375, 0.015625, 447.9, 448.0])
                        ]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    lib = O.lib()
    got_codes = np.array([lib.wtc_ref_f32_to_e4m3(float(v)) for v in x[:20000]], np.uint8)
    np.testing.assert_array_equal(got_codes, want[:20000])
    q, scale = O.quantize_e4m3_amax(x)
    assert scale == pytest.approx(np.abs(x).max() / 448.0, rel=1e-7)
    np.testing.assert_array_equal(q, torch.from_numpy(x / np.float32(scale)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy())


def test_e4m3_saturates():
    lib = O.lib()
    assert lib.wtc_ref_f32_to_e4m3(1e6) == 0x7E
    assert lib.wtc_ref_f32_to_e4m3(-1e6) == 0xFE
    assert lib.wtc_ref_f32_to_e4m3(460.0) == 0x7E


# ---------------------------------------------------------------------- chain
def _numpy_chain(a, b, scale=1.0):
    y = (a.astype(np.float64) @ b.astype(np.float64)) * scale
    e = np.exp(y - y.max(axis=1, keepdims=True))
    return y, e / e.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("m,n,k,scale", [(7, 33, 5, 1.0), (64, 128, 96, 0.3), (3, 1000, 17, -2.0)])
def test_chain_rows_against_numpy_brute_force(m, n, k, scale):
    rng = np.random.default_rng(m * n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    rows = np.arange(m)
    logits, probs = O.chain_rows(a, b, rows, scale)
    y, p = _numpy_chain(a, b, scale)
    np.testing.assert_allclose(logits, y, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(probs, p, rtol=1e-12, atol=1e-15)


def test_chain_closed_forms():
    # all-equal rows -> 1/N
    a = np.ones((4, 8), np.float32)
    b = np.full((8, 50), 0.25, np.float32)
    _, p = O.chain_rows(a, b, [0, 3])
    np.testing.assert_allclose(p, 1.0 / 50, rtol=1e-15)
    # one dominant logit -> one-hot
    b2 = np.zeros((8, 50), np.float32)
    b2[:, 17] = 100.0
    _, p2 = O.chain_rows(a, b2, [1])
    assert p2[0, 17] == pytest.approx(1.0, abs=1e-300)
    assert p2[0, :17].max() < 1e-300
    # K = 1 -> softmax of a scaled row of B
    a3 = np.float32([[2.0]])
    b3 = np.float32([[0.0, 1.0, 2.0]])
    _, p3 = O.chain_rows(a3, b3, [0])
    e = np.exp(np.array([0.0, 2.0, 4.0]) - 4.0)
    np.testing.assert_allclose(p3[0], e / e.sum(), rtol=1e-15)
    # shift invariance: adding c to every logit of a row (an extra K column of
    # A = 1 and a B row = c) leaves the softmax unchanged
    rng = np.random.default_rng(9)
    a4 = rng.standard_normal((5, 6)).astype(np.float32)
    b4 = rng.standard_normal((6, 40)).astype(np.float32)
    a5 = np.concatenate([a4, np.ones((5, 1), np.float32)], axis=1)
    b5 = np.concatenate([b4, np.full((1, 40), 3.0, np.float32)], axis=0)
    _, p4 = O.chain_rows(a4, b4, range(5))
    _, p5 = O.chain_rows(a5, b5, range(5))
    np.testing.assert_allclose(p4, p5, rtol=1e-12)


def test_chain_rows_rejects_bad_row():
    a = np.ones((2, 2), np.float32)
    with pytest.raises(ValueError):
        O.chain_rows(a, a, [2])


def test_f16_accumulate_variant_against_numpy_float16_loop():
    rng = np.random.default_rng(4)
    a = rng.uniform(-1, 1, (3, 40)).astype(np.float16).astype(np.float32)
    b = rng.uniform(-1, 1, (40, 24)).astype(np.float16).astype(np.float32)
    got = O.chain_rows_f16acc(a, b, [0, 1, 2])
    c = np.zeros((3, 24), np.float16)
    for kk in range(40):  # c = f16(c + f16(a*b)) in k order
        prod = (a[:, kk:kk + 1].astype(np.float32) * b[kk:kk + 1, :].astype(np.float32)).astype(np.float16)
        c = (c.astype(np.float32) + prod.astype(np.float32)).astype(np.float16)
    c32 = c.astype(np.float32)
    e = np.exp(c32 - c32.max(axis=1, keepdims=True))
    want = e / e.sum(axis=1, keepdims=True)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-9)
    # a scale multiplies the widened f16 logits before the softmax
    got_s = O.chain_rows_f16acc(a, b, [0, 1, 2], scale=-0.375)
    ys = c32 * np.float32(-0.375)
    e = np.exp(ys - ys.max(axis=1, keepdims=True))
    np.testing.assert_allclose(got_s, e / e.sum(axis=1, keepdims=True), rtol=2e-6, atol=1e-9)


def test_cpu_loops_baseline_matches_chain():
    rng = np.random.default_rng(5)
    a = rng.standard_normal((20, 64)).astype(np.float32)
    b = rng.standard_normal((64, 96)).astype(np.float32)
    out, secs = O.cpu_chain_loops(a, b, 4, 10, threads=2)
    _, p = O.chain_rows(a, b, range(4, 14))
    np.testing.assert_allclose(out, p, rtol=1e-4, atol=1e-7)
    assert secs >= 0.0


def test_make_inputs_quantisation_consistent():
    from welder_typical_chain_amd.configs import CONFIGS
    small = dict(m=16, n=32, k=64)
    inp = O.make_inputs(CONFIGS["C2"], seed=3, **small)
    np.testing.assert_array_equal(inp.a, O.from_f16_bits(inp.a_raw))
    inp5 = O.make_inputs(CONFIGS["C5"], seed=3, **small)
    assert inp5.a_raw.dtype == np.uint8 and inp5.scale_a > 0
    assert inp5.scale == pytest.approx(inp5.scale_a * inp5.scale_b)
    inp1 = O.make_inputs(CONFIGS["C1"], seed=0, m=8, n=8, k=8)
    np.testing.assert_array_equal(inp1.a.ravel(), O.fill_random(64, 0))  # A and B restart from the seed
    np.testing.assert_array_equal(inp1.b.ravel(), O.fill_random(64, 0))


# --------------------------------------------------------------------- golden
def test_golden_fixtures():
    """The oracle reproduces the committed vectors (tests/golden/make_golden.py)."""
    files = sorted(GOLDEN.glob("*.npz"))
    assert files, "no golden fixtures committed"
    from welder_typical_chain_amd.configs import CONFIGS
    for f in files:
        g = np.load(f, allow_pickle=False)
        cfg = CONFIGS[str(g["config"])]
        kw = {}
        for key in ("batch", "m", "n", "k"):
            if key in g.files:
                kw[key] = int(g[key])
        inp = O.make_inputs(cfg, seed=int(g["seed"]), **kw)
        assert O_checksum(inp.a_raw) == int(g["a_checksum"]), f.name
        assert O_checksum(inp.b_raw) == int(g["b_checksum"]), f.name
        rows = g["rows"]
        bt = int(g["batch_index"]) if "batch_index" in g.files else 0
        _, probs = O.chain_rows(inp.a[bt], inp.b[bt], rows, inp.scale)
        np.testing.assert_allclose(probs, g["probs"], rtol=1e-12, atol=1e-300, err_msg=f.name)


def O_checksum(arr: np.ndarray) -> int:
    """First 8 bytes of SHA-256 over the raw bytes of the quantised inputs."""
    import hashlib
    digest = hashlib.sha256(np.ascontiguousarray(arr).tobytes()).digest()
    return int.from_bytes(digest[:8], "little") >> 1
