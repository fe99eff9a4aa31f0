"""The rotation's division by f32(sqrt(head_dim)) in three operations
(lq_device.h div_sqrt_dim: q0 = y * RN(1/d), residual by one FMA, one FMA
correction; IEEE division for zeros, tiny and non-finite y), built for the
host and compared bit for bit with IEEE fp32 division over every significand
of two binades for each divisor sqrt(8) .. sqrt(512), and over the edge
cases.  Power-of-two scaling leaves the three operations exact, so the two
binades stand for every normal y above the 2^-100 threshold.  The reference
divides the rotated rows by sqrt(d) in fp32 (core/pipeline.py:49-69)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_div_sqrt_dim_matches_ieee_host(tmp_path):
    exe = tmp_path / "div_sqrt_check"
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-ffp-contract=off", "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "latticequant_amd", "csrc"), "-x", "hip", "--cuda-host-only",
                    os.path.join(ROOT, "tests", "host", "div_sqrt_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert " 0 mismatches" in r.stdout
