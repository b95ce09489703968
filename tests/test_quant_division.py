"""The quotient of the GPU quantiser's fast path (qdiv_fast in
infer_amd/csrc/iq_quant.hip) against the correctly rounded fp32 division
the reference rounds (src/quant.cpp:56-57, 70-76): an exhaustive check over
bf16 significand pairs, compiled with gcc and run on the CPU."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not found")
def test_corrected_quotient_is_the_rounded_division(tmp_path):
    exe = tmp_path / "quant_div_check"
    # -ffp-contract=off: the products and sums are the ones written
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(HERE, "cpp", "quant_div_check.c"), "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "failed_exponents 0" in out.stdout
