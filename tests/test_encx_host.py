"""The parallel chunk encoder's table entry and steps (lq_device.h encx_of,
encx_step, hull_step: k = (x + F) >> 11 from the entry's low half-word, the
base from its high half-word) built for the host and compared with the
reference's encoder step (core/gpu_ans.py:124-128) for every frequency and
every state, and the interval step with the reference step applied to every
state of the interval."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_encoder_entry_step_matches_reference_host(tmp_path):
    exe = tmp_path / "encx_check"
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-ffp-contract=off", "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "latticequant_amd", "csrc"), "-x", "hip", "--cuda-host-only",
                    os.path.join(ROOT, "tests", "host", "encx_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert " 0 mismatches" in r.stdout
