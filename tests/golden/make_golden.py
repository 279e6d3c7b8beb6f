"""Writes the golden fixtures of the CPU oracle into tests/golden/.

Each fixture records a chain configuration, the seed and extents of its
inputs, a checksum of the quantised inputs, sampled rows and the float64
softmax probabilities the oracle computes for them.  tests/test_oracle.py
checks that the oracle still reproduces them.  Run from the repository root:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402
from tests.test_oracle import O_checksum  # noqa: E402
from welder_typical_chain_amd.configs import CONFIGS  # noqa: E402

# (config, seed, extent overrides, rows, batch index)
CASES = [
    ("C1", 0, {}, np.arange(128), 0),
    ("C2", 0, {}, np.array([0, 1, 2, 3, 7, 15, 31, 63, 127, 255, 511, 1023, 2047]), 0),
    ("C3", 0, {"batch": 2}, np.array([0, 5, 1000, 2047]), 1),
    ("C4", 0, {"m": 64}, np.array([0, 17, 63]), 0),
    ("C5", 0, {"m": 256}, np.array([0, 100, 255]), 0),
]


def main() -> None:
    out = Path(__file__).resolve().parent
    for name, seed, kw, rows, bt in CASES:
        inp = O.make_inputs(CONFIGS[name], seed=seed, **kw)
        _, probs = O.chain_rows(inp.a[bt], inp.b[bt], rows, inp.scale)
        np.savez_compressed(out / f"{name.lower()}_seed{seed}.npz", config=np.array(name), seed=seed,
                            rows=rows, batch_index=bt, probs=probs,
                            a_checksum=O_checksum(inp.a_raw), b_checksum=O_checksum(inp.b_raw),
                            **{k: v for k, v in kw.items()})
        print(f"{name}: rows {len(rows)}, probs {probs.shape}")


if __name__ == "__main__":
    main()
