"""The window-score kernels' deterministic exp is the oracle's exp_det
rearranged (shifter rint, ldexp scaling, clamped argument, fixed-point add);
a C restatement of each rearranged form must give the oracle's bits.  CPU
only: builds tests/csrc/det_exp_forms.c (which includes oracle/hc_oracle.c)
with gcc and runs it on edge and random arguments."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_kernel_exp_forms_match_oracle_bit_for_bit(tmp_path):
    exe = str(tmp_path / "det_exp_forms")
    src = os.path.join(HERE, "csrc", "det_exp_forms.c")
    # no contraction: the oracle's and the kernels' sequences are separately rounded ops
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
    r = subprocess.run([exe, "4000000"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 mismatches" in r.stdout
