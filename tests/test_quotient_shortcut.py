"""The quantizers' multiply-by-reciprocal quotient shortcut, checked on the CPU in IEEE
fp32 (C, one rounding per operation) against the exact division on 2e7 random and
adversarial samples; the kernel's fp32 arithmetic is the same IEEE arithmetic."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_quotient_shortcut_matches_exact_division(tmp_path):
    exe = str(tmp_path / "quotient_shortcut_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe,
                    os.path.join(HERE, "csrc", "quotient_shortcut_check.c"), "-lm"], check=True)
    r = subprocess.run([exe, "20000000"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches=0" in r.stdout
