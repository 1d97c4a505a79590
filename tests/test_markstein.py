"""The RotorQuant kernels compute scale = m / qmax without a division
(Markstein's correction after a multiply by RN(1/qmax), see
rust-neural-network_amd/csrc/rotorquant.hip: div_qmax). This checks it against
the IEEE quotient that the reference computes (src/quant.rs:192) for every
mantissa of several binades -- the identity depends on the mantissa only away
from the overflow/underflow edges -- including the two extreme normal binades.
(A run over all 254 normal binades, 14.9 G cases, also found 0 mismatches.)"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_scale_division_is_exact(tmp_path):
    exe = tmp_path / "markstein_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-mfma", os.path.join(HERE, "markstein_check.c"),
                    "-o", str(exe), "-lm"], check=True)
    # binades of 1e-12 (the skip threshold), ~1, ~1e3, and the extremes 1 and 254
    out = subprocess.run([str(exe), "87", "127", "136", "1", "254"], check=True,
                         capture_output=True, text=True).stdout.split()
    checked, bad = int(out[0]), int(out[1])
    assert checked == 7 * 5 * (1 << 23)
    assert bad == 0


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_planted_error_is_caught(tmp_path):
    """The checker itself detects a wrong formula (q1 without the correction)."""
    src = open(os.path.join(HERE, "markstein_check.c")).read()
    broken = src.replace("fmaf(r, y, q0) : q0", "q0 : q0")
    assert broken != src
    p = tmp_path / "broken.c"
    p.write_text(broken)
    exe = tmp_path / "broken"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-mfma", str(p), "-o", str(exe), "-lm"],
                   check=True)
    out = subprocess.run([str(exe), "127"], check=True, capture_output=True, text=True).stdout.split()
    assert int(out[1]) > 0
