"""MLIR text of the Matmul -> row-Softmax chain for a ChainConfig.

Writes the chain in the dialect forms the reference's chain files use
(reference: mlir/matmul_softmax_chain_f16_native.mlir:7-95 for the decomposed
max / exp / sum / div generics, mlir/matmul_softmax_chain_named_softmax.mlir:6-21
for the named ``linalg.softmax``), extended the way the configurations need:
``linalg.batch_matmul`` for batched chains, a ``mulf`` generic by a constant
logit scale, and f32 scalar arguments for fp8 dequantisation scales.  The
compile and solver C entry points take such a file as their input.
"""
from __future__ import annotations

from .configs import ChainConfig

_ELEM = {"f32": "f32", "f16": "f16", "bf16": "bf16", "fp8": "f8E4M3FN"}


def _t(dims, elem):
    return "tensor<" + "x".join(str(d) for d in dims) + f"x{elem}>"


def _maps(rank: int, reduce_to_row: bool, nin: int) -> str:
    ds = ", ".join(f"d{i}" for i in range(rank))
    full = f"affine_map<({ds}) -> ({ds})>"
    row = f"affine_map<({ds}) -> ({', '.join(f'd{i}' for i in range(rank - 1))})>"
    maps = [full] + ([row] if nin == 2 else [])
    maps.append(row if reduce_to_row else full)
    return "[" + ", ".join(maps) + "]"


def _iters(rank: int, reduction: bool) -> str:
    its = ['"parallel"'] * (rank - 1) + ['"reduction"' if reduction else '"parallel"']
    return "[" + ", ".join(its) + "]"


def chain_mlir(cfg: ChainConfig, named_softmax: bool = False, batch: int | None = None) -> str:
    """The chain of `cfg` as MLIR text (decomposed softmax unless named_softmax)."""
    b = cfg.batch if batch is None else batch
    batched = b > 1 or cfg.name == "C3"
    lead = [b] if batched else []
    rank = len(lead) + 2
    ein, eout = _ELEM[cfg.in_dtype], _ELEM[cfg.out_dtype]
    ta = _t(lead + [cfg.m, cfg.k], ein)
    tb = _t(lead + [cfg.k, cfg.n], ein)
    tc = _t(lead + [cfg.m, cfg.n], "f32")
    tr = _t(lead + [cfg.m], "f32")
    to = _t(lead + [cfg.m, cfg.n], eout)
    fp8 = cfg.in_dtype == "fp8"
    args = f"%A: {ta}, %B: {tb}" + (", %sa: f32, %sb: f32" if fp8 else "")
    mm = "linalg.batch_matmul" if batched else "linalg.matmul"
    L = ["module {", f"  func.func @main({args}) -> {to} {{",
         "    %f0 = arith.constant 0.0 : f32",
         "    %neg_inf = arith.constant -3.4028235e+38 : f32",
         f"    %c0 = tensor.empty() : {tc}",
         f"    %c_init = linalg.fill ins(%f0 : f32) outs(%c0 : {tc}) -> {tc}",
         f"    %C0 = {mm} ins(%A, %B : {ta}, {tb}) outs(%c_init : {tc}) -> {tc}"]
    cur = "%C0"
    scale_ops = []
    if cfg.logit_scale != 1.0:
        L.append(f"    %scale = arith.constant {cfg.logit_scale!r} : f32")
        scale_ops.append("%scale")
    if fp8:
        scale_ops += ["%sa", "%sb"]
    if scale_ops:
        body = ["    ^bb0(%x: f32, %o: f32):"]
        v = "%x"
        for i, s in enumerate(scale_ops):
            body.append(f"      %y{i} = arith.mulf {v}, {s} : f32")
            v = f"%y{i}"
        body.append(f"      linalg.yield {v} : f32")
        L += [f"    %cs0 = tensor.empty() : {tc}",
              f"    %C = linalg.generic {{indexing_maps = {_maps(rank, False, 1)}, "
              f"iterator_types = {_iters(rank, False)}}} ins({cur} : {tc}) outs(%cs0 : {tc}) {{",
              *body, f"    }} -> {tc}"]
        cur = "%C"
    if named_softmax:
        L += [f"    %s0 = tensor.empty() : {tc}",
              f"    %P = linalg.softmax dimension({rank - 1}) ins({cur} : {tc}) outs(%s0 : {tc}) -> {tc}"]
    else:
        L += [f"    %m0 = tensor.empty() : {tr}",
              f"    %m_init = linalg.fill ins(%neg_inf : f32) outs(%m0 : {tr}) -> {tr}",
              f"    %max = linalg.generic {{indexing_maps = {_maps(rank, True, 1)}, "
              f"iterator_types = {_iters(rank, True)}}} ins({cur} : {tc}) outs(%m_init : {tr}) {{",
              "    ^bb0(%in: f32, %acc: f32):",
              "      %mx = arith.maximumf %in, %acc : f32",
              "      linalg.yield %mx : f32",
              f"    }} -> {tr}",
              f"    %e0 = tensor.empty() : {tc}",
              f"    %E = linalg.generic {{indexing_maps = {_maps(rank, False, 2)}, "
              f"iterator_types = {_iters(rank, False)}}} ins({cur}, %max : {tc}, {tr}) outs(%e0 : {tc}) {{",
              "    ^bb0(%x: f32, %m: f32, %o: f32):",
              "      %d = arith.subf %x, %m : f32",
              "      %e = math.exp %d : f32",
              "      linalg.yield %e : f32",
              f"    }} -> {tc}",
              f"    %s0 = tensor.empty() : {tr}",
              f"    %s_init = linalg.fill ins(%f0 : f32) outs(%s0 : {tr}) -> {tr}",
              f"    %sum = linalg.generic {{indexing_maps = {_maps(rank, True, 1)}, "
              f"iterator_types = {_iters(rank, True)}}} ins(%E : {tc}) outs(%s_init : {tr}) {{",
              "    ^bb0(%in: f32, %acc: f32):",
              "      %r = arith.addf %in, %acc : f32",
              "      linalg.yield %r : f32",
              f"    }} -> {tr}",
              f"    %p0 = tensor.empty() : {tc}",
              f"    %P = linalg.generic {{indexing_maps = {_maps(rank, False, 2)}, "
              f"iterator_types = {_iters(rank, False)}}} ins(%E, %sum : {tc}, {tr}) outs(%p0 : {tc}) {{",
              "    ^bb0(%e: f32, %s: f32, %o: f32):",
              "      %q = arith.divf %e, %s : f32",
              "      linalg.yield %q : f32",
              f"    }} -> {tc}"]
    res = "%P"
    if eout != "f32":
        L += [f"    %t0 = tensor.empty() : {to}",
              f"    %OUT = linalg.generic {{indexing_maps = {_maps(rank, False, 1)}, "
              f"iterator_types = {_iters(rank, False)}}} ins(%P : {tc}) outs(%t0 : {to}) {{",
              f"    ^bb0(%x: f32, %o: {eout}):",
              f"      %h = arith.truncf %x : f32 to {eout}",
              f"      linalg.yield %h : {eout}",
              f"    }} -> {to}"]
        res = "%OUT"
    L += [f"    return {res} : {to}", "  }", "}", ""]
    return "\n".join(L)
