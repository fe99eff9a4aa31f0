"""Build-defined subtractive dither of the rotated path (oracle side).

The reference has no E8 dither (its dithered quantizers are scalar,
ddt/dithered_comparison.py:117-147), so the oracle's lqo_dither is pinned by
what the construction must satisfy rather than by reference vectors:
SplitMix64 known answers, the dither's distribution, and the subtractive-
dither theorem: with d uniform on a fundamental domain of a sublattice of E8,
e = Q_E8(t + d) - d - t is uniform on the E8 Voronoi cell, independent of t
(per-dimension MSE G(E8) = 0.0716821, |e|^2 <= 1, the covering radius)."""
import numpy as np
import pytest

from oracle import oracle as O

M64 = (1 << 64) - 1


def _mix64_py(z):
    z = (z + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def test_splitmix64_known_answers():
    # the published SplitMix64 stream from state 0 starts 0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4
    assert O.lib().lqo_mix64(0) == 0xE220A8397B1DCDAF
    assert O.lib().lqo_mix64(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4
    rng = np.random.default_rng(0)
    for z in rng.integers(0, 2**63, 64, dtype=np.int64).tolist() + [M64, 1, 2**63]:
        assert O.lib().lqo_mix64(z) == _mix64_py(z)


def test_dither_fields_and_distribution():
    n = 1 << 18
    d = O.dither(12345, n)
    assert d.dtype == np.float32 and d.shape == (n, 8)
    assert d.min() >= -1.0 and d.max() < 1.0
    # coordinates 4p .. 4p+3 are the 16-bit fields of mix64(mix64(seed) + 2 v + p), low field first
    key = _mix64_py(12345)
    for v in (0, 1, 777, n - 1):
        for p in range(2):
            h = _mix64_py((key + 2 * v + p) & M64)
            for j in range(4):
                assert d[v, 4 * p + j] == np.float32((((h >> (16 * j)) & 0xFFFF) - (1 << 15)) * 2.0**-15)
    # every value lies on the 2^-15 grid of [-1, 1)
    assert np.array_equal(d * 2**15, np.round(d * 2**15))
    assert abs(d.mean()) < 4 * np.sqrt(1 / 3 / d.size)
    np.testing.assert_allclose(d.var(axis=0), 1 / 3, rtol=0.01)
    c = np.corrcoef(d[:, :4].T)
    assert np.abs(c - np.eye(4)).max() < 0.01
    # offset windows are consistent, seeds differ
    np.testing.assert_array_equal(O.dither(12345, 10, v0=100), d[100:110])
    assert not np.array_equal(O.dither(12346, 10), d[:10])


@pytest.mark.parametrize("sigma", [0.3, 3.9])
def test_subtractive_dither_error_is_uniform_on_voronoi_cell(sigma):
    n = 1 << 17
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((1, 1, n // 16, 128)) * sigma).astype(np.float32)
    q = O.quantize_heads(x, np.array([1.0], np.float32), dither_seed=99)
    d = O.dither(99, n)
    t = x.reshape(n, 8)
    e = (q.astype(np.float64) - d - t)
    assert (np.sum(e * e, 1) <= 1.0 + 1e-5).all()                 # inside the Voronoi cell
    np.testing.assert_allclose(np.mean(e * e), 0.0716821, rtol=0.01)   # G(E8)
    assert np.abs(e.mean(0)).max() < 0.005
    # independent of the input: no correlation, same MSE for small and large |t|
    assert abs(np.corrcoef(e[:, 0], t[:, 0])[0, 1]) < 0.01
    big = np.abs(t[:, 0]) > np.median(np.abs(t[:, 0]))
    np.testing.assert_allclose(np.mean(e[big] ** 2), np.mean(e[~big] ** 2), rtol=0.02)
    # q is an E8 point
    ok, _ = O.validate_e8(q)
    assert np.all(ok)
