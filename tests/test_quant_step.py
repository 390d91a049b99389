"""The division-free quant step of the bf16 quant kernels gives the IEEE-division result on its
whole input domain (every bf16 absmax, every bf16 value not above it), checked exhaustively on
the CPU; the GPU repeats the comparison with the device's own arithmetic
(test_quant_linear_gpu.py::test_selfcheck_quant_step)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
PAIRS = 1065402240  # bf16 pairs (a, v) with a positive finite and |v| <= a


def test_quant_step_exhaustive(tmp_path):
    exe = tmp_path / "quant_step_check"
    src = os.path.join(HERE, "quant_step_check.c")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe), src, "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=600).stdout.split()
    pairs, bad, plain = int(out[1]), int(out[3]), int(out[5])
    assert pairs == PAIRS
    assert bad == 0, f"{bad} pairs where rint of the corrected quotient differs from rint(v / s)"
    # the fma correction is needed: the bare reciprocal product rounds the wrong way on ties
    assert plain > 0
