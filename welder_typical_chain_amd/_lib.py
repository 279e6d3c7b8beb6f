"""ctypes binding of ``libwtc_hip.so`` (the C-ABI in ``include/wtc/``).

Loading fails loudly: there is no CPU or PyTorch fallback for any entry
point.  Build the library first (``python -m welder_typical_chain_amd.build``).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libwtc_hip.so"

WTC_OK = 0
WTC_ERR_ARG = 1
WTC_ERR_WORKSPACE = 2
WTC_ERR_HIP = 3
WTC_ERR_UNSUPPORTED = 4
WTC_ERR_TIMEOUT = 5
NOALLOC_SCRATCH_BYTES = 8 << 20

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_FP8_E4M3 = 3

PATH_AUTO = 0
PATH_EXCHANGE = 1
PATH_SPLIT = 2
PATH_UNFUSED = 3
PATH_ROWS = 4

PATHS = {"auto": PATH_AUTO, "exchange": PATH_EXCHANGE, "split": PATH_SPLIT,
         "unfused": PATH_UNFUSED, "rows": PATH_ROWS}

_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p


class Tiles(ctypes.Structure):
    """wtc_tiles: the five best.json tile parameters of a kernel variant."""
    _fields_ = [("tile_m", _c_i64), ("tile_n", _c_i64), ("tile_k", _c_i64),
                ("thread_tile_m", _c_i64), ("thread_tile_n", _c_i64)]

    def as_list(self):
        return [self.tile_m, self.tile_n, self.tile_k, self.thread_tile_m, self.thread_tile_n]


_c_tiles = ctypes.POINTER(Tiles)

# name -> (restype, argtypes); every symbol the headers under include/wtc declare.
SIGNATURES = {
    "wtc_matmul_softmax": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                          ctypes.c_float, ctypes.c_float, ctypes.c_int,
                                          _c_p, ctypes.c_size_t, _c_p]),
    "wtc_matmul_softmax_noalloc": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                                  ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                                  ctypes.c_float, ctypes.c_float, ctypes.c_int, _c_p]),
    "wtc_matmul_softmax_tiles": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                                ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                                ctypes.c_float, ctypes.c_float, _c_tiles,
                                                ctypes.c_int, _c_p, ctypes.c_size_t, _c_p]),
    "wtc_profile_tiles": (ctypes.c_int, [_c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, ctypes.c_int,
                                         _c_tiles, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_uint64, ctypes.POINTER(ctypes.c_double)]),
    "wtc_list_variants": (ctypes.c_int, [ctypes.c_int, _c_tiles, ctypes.POINTER(ctypes.c_uint),
                                         ctypes.POINTER(ctypes.c_char_p), ctypes.c_int]),
    "wtc_plan_tiles": (ctypes.c_int, [_c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, _c_tiles, ctypes.c_int, ctypes.c_int, _c_tiles,
                                      ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_c_i64),
                                      ctypes.POINTER(_c_i64), ctypes.POINTER(ctypes.c_double)]),
    "wtc_matmul_softmax_workspace_size": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64,
                                                   ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "wtc_workspace_init": (ctypes.c_int, [_c_p, ctypes.c_size_t, _c_p]),
    "wtc_plan": (ctypes.c_int, [_c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, ctypes.c_int,
                                ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                ctypes.POINTER(_c_i64), ctypes.POINTER(ctypes.c_int),
                                ctypes.POINTER(_c_i64)]),
    "wtc_read_error_flags": (ctypes.c_int, [_c_p, ctypes.POINTER(ctypes.c_uint32), ctypes.c_int]),
    "wtc_check_status": (ctypes.c_int, [_c_p]),
    "wtc_set_exchange_wait_limit": (ctypes.c_int, [ctypes.c_uint64]),
    "wtc_release_stream": (ctypes.c_int, [_c_p]),
    "wtc_last_error": (ctypes.c_char_p, []),
    "wtc_version": (ctypes.c_char_p, []),
    "welder_compile_typical_chain_to_nvvm": (ctypes.c_int, [
        ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, ctypes.c_int,
        ctypes.c_char_p, ctypes.c_size_t]),
    "welder_compile_typical_chain_to_hip": (ctypes.c_int, [
        ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, ctypes.c_int,
        ctypes.c_char_p, ctypes.c_size_t]),
    "welder_solver_solve_typical_chain": (ctypes.c_int, [
        ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _c_i64, ctypes.c_int,
        ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64),
        ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), ctypes.c_char_p, ctypes.c_size_t]),
}

_lib = None
_stamps_lib = None


class WtcError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"wtc error {code}: {msg}")
        self.code = code


def _load(path: Path) -> ctypes.CDLL:
    if not path.exists():
        raise RuntimeError(
            f"{path} is missing: the HIP extension is not built "
            "(run python -m welder_typical_chain_amd.build); no fallback exists")
    # PyTorch ships its own HIP runtime (torch/lib/libamdhip64.so, soname
    # libamdhip64.so.7) and asks for it as "libamdhip64.so".  Loaded first,
    # it satisfies this library's libamdhip64.so.7 dependency, so one
    # runtime serves both.  Loaded the other way round, the process would
    # hold two HIP runtimes and the second one finds no device.
    import torch  # noqa: F401
    h = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(h, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    return h


def lib() -> ctypes.CDLL:
    """The loaded library with every declared signature bound."""
    global _lib
    if _lib is None:
        _lib = _load(LIB_PATH)
    return _lib


def stamps_lib() -> ctypes.CDLL:
    """The profiling build with the exchange kernel's phase stamps
    (libwtc_hip_stamps.so): the same C-ABI plus wtc_phase_stamps_read."""
    global _stamps_lib
    if _stamps_lib is None:
        h = _load(LIB_PATH.with_name("libwtc_hip_stamps.so"))
        h.wtc_phase_stamps_read.restype = ctypes.c_int
        h.wtc_phase_stamps_read.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_int64]
        _stamps_lib = h
    return _stamps_lib


def check(code: int) -> None:
    if code != WTC_OK:
        raise WtcError(code, lib().wtc_last_error().decode())


def variants(in_dtype: int):
    """[(name, [tileM, tileN, tileK, threadTileM, threadTileN], paths bitmask)]
    of the kernel variants built for an input type (wtc_list_variants)."""
    L = lib()
    count = L.wtc_list_variants(in_dtype, None, None, None, 0)
    if count < 0:
        check(WTC_ERR_ARG)
    tiles = (Tiles * count)()
    paths = (ctypes.c_uint * count)()
    names = (ctypes.c_char_p * count)()
    L.wtc_list_variants(in_dtype, tiles, paths, names, count)
    return [(names[i].decode(), tiles[i].as_list(), int(paths[i])) for i in range(count)]


def plan(batch: int, m: int, n: int, k: int, in_dtype: int, out_dtype: int, path: int = PATH_AUTO,
         tiles=None, cu_count: int = 256, wg_per_cu: int = 1) -> dict:
    """wtc_plan_tiles: the variant and path the cost model picks, with its
    grid, workspace bytes and estimated microseconds per call."""
    chosen = Tiles()
    cpath = ctypes.c_int()
    grid = ctypes.c_int64()
    ws = ctypes.c_int64()
    est = ctypes.c_double()
    want = Tiles(*tiles) if tiles is not None else None
    rc = lib().wtc_plan_tiles(batch, m, n, k, in_dtype, out_dtype, path,
                              ctypes.byref(want) if want is not None else None, cu_count, wg_per_cu,
                              ctypes.byref(chosen), ctypes.byref(cpath), ctypes.byref(grid),
                              ctypes.byref(ws), ctypes.byref(est))
    check(rc)
    return {"tiles": chosen.as_list(), "path": cpath.value, "grid": grid.value,
            "workspace_bytes": ws.value, "est_us": est.value}
