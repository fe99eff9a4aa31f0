"""The rotation's division by f32(sqrt(head_dim)) in three operations
(lq_device.h div_sqrt_dim: q0 = y * RN(1/d), residual by one FMA, one FMA
correction; IEEE division for zeros, tiny and non-finite y), built for the
host and compared bit for bit with IEEE fp32 division over every significand
of two binades for each divisor sqrt(8) .. sqrt(512), and over the edge
cases.  Power-of-two scaling leaves the three operations exact, so the two
binades stand for every normal y above the 2^-100 threshold.  The reference
divides the rotated rows by sqrt(d) in fp32 (core/pipeline.py:49-69).

Also the rotated quantizer's division of the rotated rows by the per-head
scale (lq_device.h div_exact: two Markstein corrections of RN(x * RN(1/s)),
for |x| and s in [2^-60, 2^60]), compared bit for bit with IEEE division
over every significand of x for the divisors whose reciprocal rounds worst,
random divisors, and every pair of binades in the range
(llm/compressed_kv_cache.py:199-201 divides by the scale in fp32)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _host_fma():
    """-mfma where the host CPU has it (hardware fmaf instead of the library's)."""
    try:
        with open("/proc/cpuinfo") as f:
            return ["-mfma"] if " fma " in f.read() else []
    except OSError:
        return []


def _run_check(tmp_path, name):
    exe = tmp_path / name
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", *_host_fma(),
                    "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "latticequant_amd", "csrc"), "-x", "hip", "--cuda-host-only",
                    os.path.join(ROOT, "tests", "host", name + ".cpp"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert " 0 mismatches" in r.stdout


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_div_sqrt_dim_matches_ieee_host(tmp_path):
    _run_check(tmp_path, "div_sqrt_check")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_div_exact_matches_ieee_host(tmp_path):
    _run_check(tmp_path, "div_exact_check")
