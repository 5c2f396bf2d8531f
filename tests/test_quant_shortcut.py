"""CPU: the exact-division shortcut of the int8 archive kernel's scale
(fl(absmax / 127) from a reciprocal product and one fma correction) agrees
with IEEE division for every non-negative finite float."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_div127_shortcut_exhaustive(tmp_path):
    exe = str(tmp_path / "qchk")
    src = os.path.join(HERE, "quant_shortcut_check.c")
    # -ffp-contract=off: no fusing beyond the explicit fmaf calls
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", src, "-o", exe, "-lm"],
                   check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True,
                         env={**os.environ, "OMP_NUM_THREADS": str(min(8, os.cpu_count() or 1))})
    n, bad = map(int, out.stdout.split())
    assert n == 0x7F800000 and bad == 0
