"""The FP8 row quantiser's division shortcut (csrc/fp8_quant.hip: div_sc -- a reciprocal, a product and one FMA
correction step) against IEEE division, on the CPU: every finite bf16 value against 2048 scales and 2e7 random fp32
pairs, wherever the quotient can reach an e4m3 value. The GPU tests then pin the quantiser's bytes against the
oracle; this pins the arithmetic identity they rely on for inputs those tests do not draw."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fma_corrected_division_equals_ieee(tmp_path):
    exe = str(tmp_path / "fp8_division_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, os.path.join(HERE, "fp8_division_check.c"),
                    "-lm"], check=True)
    res = subprocess.run([exe, "2048", "20000000"], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "mismatches 0" in res.stdout
