"""The fp32 quotient of the QDQ kernels (rx-met_amd/csrc/div_rn.h, Markstein's correction of
x times the correctly rounded reciprocal) equals IEEE division wherever the kernels take it:
tests/div_rn_check.c compiled with gcc (fma from the C library, no contraction) over every
1021st fp32 bit pattern for 24 scales.  The full sweep (every pattern) was run the same way.
The kernels' own quotients are compared with numpy's on the GPU in
tests/test_qdq_gpu.py::test_quotients_are_correctly_rounded."""
import shutil
import subprocess
from pathlib import Path

import pytest


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_markstein_quotient_equals_ieee_division(tmp_path):
    src = Path(__file__).with_name("div_rn_check.c")
    exe = tmp_path / "div_rn_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(src), "-lm"], check=True)
    r = subprocess.run([str(exe), "1021"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:]
    assert "TOTAL bad=0" in r.stdout
