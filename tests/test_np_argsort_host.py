"""numpy.argsort tie order as the table kernels restate it (lq_argsort.h),
built for the host with one lane and compared with numpy.argsort itself.

build_rans_table ranks symbols with np.argsort(-counts) / np.argsort(-freqs)
(reference core/gpu_ans.py:76,80); numpy's argsort is not stable, so the
order inside a tie group decides which frequencies the adjustment loop
changes.  The restatement covers every alphabet size a table can have
(n <= 1028): the 8-lane bitonic network (n <= 256), the 4-register unrolled
quicksort partition above it, and the std::sort fallback that runs once the
quicksort's depth budget is spent (a pivot equal to the range minimum).
The fallback is also compared with libstdc++'s std::sort directly, on inputs
that include McIlroy's adversary, which drives introsort into heap sort.

numpy's order is that of the host it runs on (x86-simd-sort on AVX-512);
the check is skipped on hosts without AVX-512, where numpy sorts another way.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _avx512():
    from numpy._core._multiarray_umath import __cpu_features__ as f
    return bool(f.get("AVX512_SKX"))


pytestmark = [pytest.mark.skipif(not _avx512(), reason="numpy sorts without AVX-512 on this host"),
              pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")]


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    so = tmp_path_factory.mktemp("npsort") / "np_argsort_host.so"
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "latticequant_amd", "csrc"), "-x", "hip", "--cuda-host-only",
                    os.path.join(ROOT, "tests", "host", "np_argsort_host.cpp"), "-o", str(so)],
                   check=True, capture_output=True)
    lib = ctypes.CDLL(str(so))
    lib.np_argsort_host.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    lib.np_argsort_host.restype = ctypes.c_int
    lib.np_std_sort_check.argtypes = [ctypes.c_uint64, ctypes.c_long]
    lib.np_std_sort_check.restype = ctypes.c_long
    return lib


def _restated(lib, k):
    k = np.ascontiguousarray(k, dtype=np.int64)
    out = np.empty(len(k), np.int64)
    assert lib.np_argsort_host(k.ctypes.data, out.ctypes.data, len(k)) == 0
    return out


def _keys(rng, n, kind):
    if kind == 0:
        return -rng.integers(0, 4, n)                       # few distinct counts
    if kind == 1:
        return -rng.geometric(0.05, n)                      # geometric counts
    if kind == 2:                                           # minimum-dominated: the std::sort fallback
        k = -rng.integers(0, 3, n)
        k[rng.random(n) < 0.7] = -50
        return k
    if kind == 3:
        return -np.minimum(rng.pareto(1.0, n).astype(np.int64), 5000)
    if kind == 4:                                           # -freqs after a normalisation
        c = rng.geometric(0.01, n)
        return -np.maximum((c / c.sum() * 1024).astype(np.int64), 1)
    if kind == 5:                                           # histogram of a heavy-tailed symbol stream
        s = np.round(rng.standard_t(3, 4000) * rng.uniform(5, 60)).astype(np.int64)
        c = np.bincount(s - s.min() + 2, minlength=n + 4)
        return -c[:n]
    return -rng.integers(0, 2, n)                           # two values


def test_np_argsort_matches_numpy_host(lib):
    rng = np.random.default_rng(20260)
    cases, bad, wide = 100_000, 0, 0
    for t in range(cases):
        n = int(rng.integers(257, 1029)) if t % 4 else int(rng.integers(0, 257))
        k = _keys(rng, n, t % 7)
        wide += n > 256
        if not np.array_equal(_restated(lib, k), np.argsort(k)):
            bad += 1
    assert wide >= 70_000
    assert bad == 0, f"{bad} of {cases} orders differ from numpy.argsort"


def test_np_argsort_edge_sizes_host(lib):
    rng = np.random.default_rng(7)
    for n in (0, 1, 2, 7, 8, 9, 255, 256, 257, 288, 289, 511, 512, 513, 1023, 1024, 1028):
        for kind in range(7):
            k = _keys(rng, n, kind)
            np.testing.assert_array_equal(_restated(lib, k), np.argsort(k), err_msg=f"n={n} kind={kind}")
        z = np.zeros(n, np.int64)   # all equal
        np.testing.assert_array_equal(_restated(lib, z), np.argsort(z))


def test_std_sort_fallback_matches_libstdcxx_host(lib):
    assert lib.np_std_sort_check(1, 20000) == 0
