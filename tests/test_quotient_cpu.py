"""The quantiser quotient of the HIP kernels (gdnr_device.h, quotient_rn) is
the correctly rounded IEEE quotient x / s on every block it is used for.

The kernels replace the division in the requantisation with x * RN(1/s) and
two Newton corrections whose residuals are exact by FMA (Markstein's
theorem); this compiles the same operation sequence in C with glibc's exact
fmaf and compares it bit for bit with x / s on random quantiser-shaped
blocks and on adversarial divisors and dividends. The device side of the same
claim is tests/test_gpu_parity.py::test_quantizer_bit_exact.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_quotient_rn_equals_ieee_division(tmp_path):
    exe = tmp_path / "quotient_rn_check"
    # -ffp-contract=off: the C statements must round exactly as the device's
    # separate multiply and fused multiply-adds do
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", str(HERE / "quotient_rn_check.c"), "-o", str(exe), "-lm"],
                   check=True)
    res = subprocess.run([str(exe), "4000000", "2000"], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert " 0 mismatches" in res.stdout
