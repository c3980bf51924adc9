"""The quantizer's reciprocal + FMA-correction division gives the IEEE codes.

Compiles tests/exhaustive_division.c with gcc and checks every (x, amax)
pair of 16-bit inputs (bf16: 1.8e9 pairs, about 11 s on 8 cores; f16: 1.5e9
pairs, about 2 s). ACTUNE_DIVISION_STRIDE=n samples every n-th amax.
"""
import os
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
SRC = HERE / "exhaustive_division.c"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("div") / "exhaustive_division"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", str(SRC), "-o", str(exe), "-lm"], check=True)
    return exe


@pytest.mark.parametrize("fmt", ["bf16", "f16"])
def test_fast_division_codes_match_ieee(checker, fmt):
    stride = os.environ.get("ACTUNE_DIVISION_STRIDE", "1")
    res = subprocess.run([str(checker), fmt, stride], capture_output=True, text=True, timeout=600)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    assert "mismatches 0" in res.stdout
