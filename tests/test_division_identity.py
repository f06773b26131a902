"""The prepass's fixed-divisor quotient (product + one FMA correction with the
correctly rounded reciprocal) equals IEEE division over the quotient range the
E4M3 encoding can see.  A reduced sweep of tests/native/div_identity.c; the
full sweep (mantissa stride 7, 400 scales: 2.1e10 cases) also passes."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fixed_divisor_quotient_is_ieee(tmp_path):
    exe = tmp_path / "div_identity"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", os.path.join(HERE, "native", "div_identity.c"), "-o",
                    str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe), "997", "120"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
