"""Exhaustive pin of the quantizer's division shortcut used by the gfx950 kernels.

model/int8.py:66-67 divides by the row scale; the kernels multiply by its
reciprocal and apply one fma correction, or (the fused norm, absmax < 2^80)
multiply by a two-term reciprocal. tests/quant_division_check.c compares each
with the division on every bf16 (absmax, x) pair with |x| <= absmax.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_corrected_reciprocal_quotient_matches_division_exhaustively(tmp_path):
    exe = tmp_path / "quant_division_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp",
                    os.path.join(HERE, "quant_division_check.c"), "-lm", "-o", str(exe)], check=True)
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(16, os.cpu_count() or 1)))
    out = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    fields = out.stdout.split()
    cases, diffs, plain = int(fields[1]), int(fields[3]), int(fields[5])
    split_cases, split_diffs = int(fields[7]), int(fields[9])
    assert cases == 1_065_402_238          # all positive finite bf16 absmax x all |x| <= absmax, +-
    assert diffs == 0, out.stdout
    assert plain > 0                       # the uncorrected reciprocal alone would not do
    assert split_cases == 702_064_510 and split_diffs == 0, out.stdout   # every absmax < 2^80
    assert out.returncode == 0
