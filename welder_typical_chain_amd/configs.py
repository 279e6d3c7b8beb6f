"""The five workloads of the chain (shapes, element types, input laws).

C1 is the reference's own CPU-runnable chain (mlir/matmul_softmax_chain.mlir
at 128^3 with the profiler's xorshift32 uniform[-1,1] inputs); C2-C5 are the
MI355X workloads.  C2 is the headline configuration.
"""
from __future__ import annotations

import math
from dataclasses import dataclass


@dataclass(frozen=True)
class ChainConfig:
    name: str
    batch: int
    m: int
    n: int
    k: int
    in_dtype: str        # "f32" | "f16" | "bf16" | "fp8"
    out_dtype: str       # "f32" | "f16" | "bf16"
    dist: str            # "xorshift_uniform" | "normal" | "uniform"
    dist_param: float    # stddev for "normal", half-width for "uniform"
    logit_scale: float = 1.0
    description: str = ""

    @property
    def flops(self) -> int:
        return 2 * self.batch * self.m * self.n * self.k

    def bytes_moved(self) -> int:
        isz = {"f32": 4, "f16": 2, "bf16": 2, "fp8": 1}[self.in_dtype]
        osz = {"f32": 4, "f16": 2, "bf16": 2}[self.out_dtype]
        return self.batch * ((self.m * self.k + self.k * self.n) * isz + self.m * self.n * osz)


C1 = ChainConfig("C1", 1, 128, 128, 128, "f32", "f32", "xorshift_uniform", 1.0,
                 description="f32 chain, A[128x128] x B[128x128], uniform[-1,1] xorshift32 seed 0")
C2 = ChainConfig("C2", 1, 2048, 2048, 1024, "f16", "f16", "normal", 1.0 / math.sqrt(1024),
                 description="f16 chain, A[2048x1024] x B[1024x2048], N(0,1)/sqrt(K), f16 out")
C3 = ChainConfig("C3", 64, 2048, 2048, 128, "f16", "f16", "normal", 1.0,
                 logit_scale=1.0 / math.sqrt(128),
                 description="attention scores, Q[64x2048x128] x K^T[64x128x2048], scale 1/sqrt(128)")
C4 = ChainConfig("C4", 1, 1024, 32768, 4096, "bf16", "f16", "uniform", 0.5,
                 description="wide-row logits, bf16 A[1024x4096] x B[4096x32768], split-N softmax")
C5 = ChainConfig("C5", 1, 8192, 8192, 4096, "fp8", "f16", "normal", 1.0,
                 description="fp8 e4m3 A[8192x4096] x B[4096x8192], per-tensor amax scales, f16 out")

CONFIGS = {c.name: c for c in (C1, C2, C3, C4, C5)}
HEADLINE = C2
