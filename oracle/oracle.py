"""numpy / ctypes face of the CPU oracle (oracle/wtc_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker and by bench.py's cpu_baseline leg; never by the product path.
Each function notes which reference behaviour it restates (file:line in the
reference repository); the C source notes how each is pinned.
"""
from __future__ import annotations

import ctypes
import subprocess
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libwtc_oracle.so"
# the same source built with ROCm's clang -O3 and LLVM's OpenMP: the loops
# bench.py times as the CPU baseline
BASELINE_LIB_PATH = HERE / "_build" / "libwtc_cpu_baseline.so"

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_f64p = ctypes.POINTER(ctypes.c_double)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i64 = ctypes.c_int64

_SIGS = {
    "wtc_ref_xorshift32": (ctypes.c_uint32, [ctypes.c_uint32]),
    "wtc_ref_fill_random_f32": (None, [_f32p, _i64, ctypes.c_uint64]),
    "wtc_ref_fill_linear_f32": (None, [_f32p, _i64]),
    "wtc_ref_fill_uniform_f32": (None, [_f32p, _i64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]),
    "wtc_ref_fill_normal_f32": (None, [_f32p, _i64, ctypes.c_uint64, ctypes.c_float]),
    "wtc_ref_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "wtc_ref_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "wtc_ref_f32_to_f16_profiler": (ctypes.c_uint16, [ctypes.c_float]),
    "wtc_ref_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
    "wtc_ref_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "wtc_ref_f32_to_e4m3": (ctypes.c_uint8, [ctypes.c_float]),
    "wtc_ref_e4m3_to_f32": (ctypes.c_float, [ctypes.c_uint8]),
    "wtc_ref_quantize_f16": (None, [_f32p, _u16p, _i64]),
    "wtc_ref_quantize_bf16": (None, [_f32p, _u16p, _i64]),
    "wtc_ref_quantize_e4m3_amax": (ctypes.c_float, [_f32p, _u8p, _i64]),
    "wtc_ref_dequant_f16": (None, [_u16p, _f32p, _i64]),
    "wtc_ref_dequant_bf16": (None, [_u16p, _f32p, _i64]),
    "wtc_ref_dequant_e4m3": (None, [_u8p, _f32p, _i64]),
    "wtc_ref_chain_rows": (ctypes.c_int, [_f32p, _f32p, _i64, _i64, _i64, _i64p, _i64,
                                          ctypes.c_double, _f64p, _f64p]),
    "wtc_ref_chain_rows_f16acc": (ctypes.c_int, [_f32p, _f32p, _i64, _i64, _i64, _i64p, _i64,
                                                  ctypes.c_float, _f64p]),
    "wtc_cpu_chain_loops_f32": (ctypes.c_double, [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64,
                                                  _i64, ctypes.c_int]),
    "wtc_cpu_max_threads": (ctypes.c_int, []),
}


def build() -> Path:
    """Compile oracle/wtc_oracle.c with its Makefile (always)."""
    subprocess.run(["make", "-B", "-C", str(HERE)], check=True, capture_output=True)
    return LIB_PATH


def _load(path: Path) -> ctypes.CDLL:
    if not path.exists():
        build()
    h = ctypes.CDLL(str(path))
    for name, (res, args) in _SIGS.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    return h


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load(LIB_PATH)
    return _lib


_baseline_lib = None


def baseline_lib() -> ctypes.CDLL:
    """The clang -O3 build (CPU baseline timing only)."""
    global _baseline_lib
    if _baseline_lib is None:
        _baseline_lib = _load(BASELINE_LIB_PATH)
    return _baseline_lib


def _p(arr: np.ndarray, ptype):
    assert arr.flags["C_CONTIGUOUS"]
    return arr.ctypes.data_as(ptype)


# ---------------------------------------------------------------- generators
def fill_random(n: int, seed: int) -> np.ndarray:
    """--init=random (WelderProfilerRuntime.h:141-149): xorshift32 uniform[-1,1] in f32."""
    out = np.empty(n, np.float32)
    lib().wtc_ref_fill_random_f32(_p(out, _f32p), n, seed)
    return out


def fill_linear(n: int) -> np.ndarray:
    """--init=linear (WelderProfilerRuntime.h:136-139)."""
    out = np.empty(n, np.float32)
    lib().wtc_ref_fill_linear_f32(_p(out, _f32p), n)
    return out


def fill_uniform(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().wtc_ref_fill_uniform_f32(_p(out, _f32p), n, seed, lo, hi)
    return out


def fill_normal(n: int, seed: int, std: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().wtc_ref_fill_normal_f32(_p(out, _f32p), n, seed, std)
    return out


# ------------------------------------------------------------------ formats
def to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape, np.uint16)
    lib().wtc_ref_quantize_f16(_p(x, _f32p), _p(q, _u16p), x.size)
    return q


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape, np.uint16)
    lib().wtc_ref_quantize_bf16(_p(x, _f32p), _p(q, _u16p), x.size)
    return q


def quantize_e4m3_amax(x: np.ndarray) -> tuple[np.ndarray, float]:
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape, np.uint8)
    scale = lib().wtc_ref_quantize_e4m3_amax(_p(x, _f32p), _p(q, _u8p), x.size)
    return q, float(scale)


def from_f16_bits(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint16)
    x = np.empty(q.shape, np.float32)
    lib().wtc_ref_dequant_f16(_p(q, _u16p), _p(x, _f32p), q.size)
    return x


def from_bf16_bits(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint16)
    x = np.empty(q.shape, np.float32)
    lib().wtc_ref_dequant_bf16(_p(q, _u16p), _p(x, _f32p), q.size)
    return x


def from_e4m3(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    x = np.empty(q.shape, np.float32)
    lib().wtc_ref_dequant_e4m3(_p(q, _u8p), _p(x, _f32p), q.size)
    return x


# -------------------------------------------------------------------- chain
def chain_rows(a: np.ndarray, b: np.ndarray, rows, scale: float = 1.0):
    """float64 softmax_row(scale * a @ b) on the selected rows (one batch).

    Chain semantics of mlir/matmul_softmax_chain.mlir:10-83 and the verifier's
    closed form backend/welder/bench/verify_matmul_softmax.py:242-261.
    Returns (logits, probs), each [len(rows), N] float64.
    """
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    rows = np.ascontiguousarray(np.asarray(rows, np.int64))
    logits = np.empty((rows.size, n), np.float64)
    probs = np.empty((rows.size, n), np.float64)
    rc = lib().wtc_ref_chain_rows(_p(a, _f32p), _p(b, _f32p), m, n, k, _p(rows, _i64p),
                                  rows.size, scale, _p(logits, _f64p), _p(probs, _f64p))
    if rc:
        raise ValueError(f"wtc_ref_chain_rows failed ({rc})")
    return logits, probs


def chain_rows_f16acc(a: np.ndarray, b: np.ndarray, rows, scale: float = 1.0) -> np.ndarray:
    """The reference lowering's f16-accumulate chain (information only):
    f16 accumulation in k order, widened to f32, times `scale`, f32 softmax."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    _, n = b.shape
    rows = np.ascontiguousarray(np.asarray(rows, np.int64))
    probs = np.empty((rows.size, n), np.float64)
    rc = lib().wtc_ref_chain_rows_f16acc(_p(a, _f32p), _p(b, _f32p), m, n, k, _p(rows, _i64p),
                                         rows.size, float(scale), _p(probs, _f64p))
    if rc:
        raise ValueError("wtc_ref_chain_rows_f16acc failed")
    return probs


def cpu_chain_loops(a: np.ndarray, b: np.ndarray, row0: int, nrows: int, threads: int = 1,
                    baseline: bool = False):
    """The chain lowered to loops in f32 on rows [row0, row0+nrows); returns
    (out, seconds).  baseline=True runs the clang -O3 build."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    k = a.shape[1]
    n = b.shape[1]
    c = np.empty((nrows, n), np.float32)
    out = np.empty((nrows, n), np.float32)
    h = baseline_lib() if baseline else lib()
    secs = h.wtc_cpu_chain_loops_f32(_p(a, _f32p), _p(b, _f32p), _p(c, _f32p), _p(out, _f32p),
                                     n, k, row0, nrows, threads)
    return out, float(secs)


def cpu_max_threads(baseline: bool = False) -> int:
    return int((baseline_lib() if baseline else lib()).wtc_cpu_max_threads())


# ------------------------------------------------------------------- inputs
@dataclass
class ChainInputs:
    """Quantised inputs as the GPU consumes them, and their f32 decoding."""
    a_raw: np.ndarray   # float32 / uint16 (f16 or bf16 bits) / uint8 (e4m3)
    b_raw: np.ndarray
    a: np.ndarray       # f32 decoding, same shape
    b: np.ndarray
    scale_a: float
    scale_b: float
    logit_scale: float

    @property
    def scale(self) -> float:
        """Multiplier of a @ b before the softmax."""
        return self.logit_scale * self.scale_a * self.scale_b


def seed_b(seed: int) -> int:
    """Seed of B's stream: seed + golden-ratio constant mod 2^32 (never 0 or 1,
    which xorshift32 treats alike, for small seeds)."""
    return (int(seed) + 0x9E3779B1) & 0xFFFFFFFF


def make_inputs(cfg, seed: int = 0, batch: int | None = None, m: int | None = None,
                n: int | None = None, k: int | None = None) -> ChainInputs:
    """Seeded inputs of a chain config (optionally with overridden extents).

    xorshift_uniform: the reference profiler's --init=random, A and B each
      restarting from the seed (WelderProfilerRuntime.h:141); f32.
    normal / uniform: this build's generators, A from `seed`, B from
      `seed_b(seed)` (a different xorshift32 stream).
    Quantisation: f16 / bf16 round to nearest even; fp8 per-tensor amax e4m3.
    """
    batch = cfg.batch if batch is None else batch
    m = cfg.m if m is None else m
    n = cfg.n if n is None else n
    k = cfg.k if k is None else k
    na, nb = batch * m * k, batch * k * n
    if cfg.dist == "xorshift_uniform":
        af, bf = fill_random(na, seed), fill_random(nb, seed)
    elif cfg.dist == "normal":
        af, bf = fill_normal(na, seed, cfg.dist_param), fill_normal(nb, seed_b(seed), cfg.dist_param)
    elif cfg.dist == "uniform":
        h = cfg.dist_param
        af, bf = fill_uniform(na, seed, -h, h), fill_uniform(nb, seed_b(seed), -h, h)
    else:
        raise ValueError(cfg.dist)
    shape_a = (batch, m, k)
    shape_b = (batch, k, n)
    sa = sb = 1.0
    if cfg.in_dtype == "f32":
        a_raw, b_raw = af, bf
        a_dec, b_dec = af, bf
    elif cfg.in_dtype == "f16":
        a_raw, b_raw = to_f16_bits(af), to_f16_bits(bf)
        a_dec, b_dec = from_f16_bits(a_raw), from_f16_bits(b_raw)
    elif cfg.in_dtype == "bf16":
        a_raw, b_raw = to_bf16_bits(af), to_bf16_bits(bf)
        a_dec, b_dec = from_bf16_bits(a_raw), from_bf16_bits(b_raw)
    elif cfg.in_dtype == "fp8":
        a_raw, sa = quantize_e4m3_amax(af)
        b_raw, sb = quantize_e4m3_amax(bf)
        a_dec, b_dec = from_e4m3(a_raw), from_e4m3(b_raw)
    else:
        raise ValueError(cfg.in_dtype)
    return ChainInputs(a_raw.reshape(shape_a), b_raw.reshape(shape_b), a_dec.reshape(shape_a),
                       b_dec.reshape(shape_b), sa, sb, cfg.logit_scale)
