"""The quantizer's nearest-point search (lq_device.h e8_nearest_fast: a
margin-checked estimate of the coset distance difference, with the
reference-order sums as the fallback) built for the host and run against the
CPU oracle's encode_e8 (core/e8_quantizer.py:20-83) on 16M random and
adversarial vectors: Gaussian at many scales, near-ties of the two cosets,
exact dyadic ties, mixed magnitudes, perturbed half-integers.  The same
function is what the gfx950 kernels run; the GPU parity tests cover it there."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_e8_fast_search_matches_oracle_host(tmp_path):
    gcc = shutil.which("gcc")
    assert gcc, "gcc is required to build the oracle object"
    obj = tmp_path / "lq_oracle.o"
    subprocess.run([gcc, "-O2", "-c", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
                    os.path.join(ROOT, "oracle", "lq_oracle.c"), "-o", str(obj)], check=True)
    exe = tmp_path / "e8_fast_check"
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-ffp-contract=off", "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "latticequant_amd", "csrc"), "-x", "hip", "--cuda-host-only",
                    os.path.join(ROOT, "tests", "host", "e8_fast_check.cpp"), "-x", "none", str(obj),
                    "-o", str(exe), "-lpthread"], check=True, capture_output=True)
    r = subprocess.run([str(exe), "2000000"], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert "0 mismatches" in r.stdout
