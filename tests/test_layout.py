"""CPU replay of the kernel's index maps (tests/layout_check.cpp): one
workgroup's data movement through the LDS swizzles and the MFMA fragment /
accumulator layouts must reproduce a plain integer matmul; the XCD-aware
workgroup-to-tile map must be a bijection."""
from __future__ import annotations

import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_layout_replay(tmp_path):
    exe = tmp_path / "layout_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", f"-I{ROOT / 'welder_typical_chain_amd' / 'csrc'}",
                    str(ROOT / "tests" / "layout_check.cpp"), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip().splitlines()[-1] == "OK"
