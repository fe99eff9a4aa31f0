"""Regenerate the inputs behind the reference-written fixtures that store
only their outputs, by replaying make_golden.py's numpy RNG sequence (no
reference code is run).  Data helper for the tests."""
import numpy as np

from oracle import oracle as O


def compact_inputs():
    """The 6000 x 8 inputs behind compact.npz's inrange{b} masks, regenerated
    by replaying tests/golden/make_golden.py's numpy RNG sequence (seed
    20261201: the E8 inputs are drawn first, then per rate 6000 Gaussian rows
    and 3000 x b raw bytes), then x / a (a = compute_scale(1, b)) in fp32."""
    rng = np.random.default_rng(20261201)
    for b in (3, 4, 5):
        rng.standard_normal((4096, 8))
    rng.standard_normal((2048, 8))
    rng.integers(-16, 17, size=(4096, 8))
    rng.integers(-8, 9, size=(2048, 8))
    rng.integers(-4, 5, size=(2048, 8))
    rng.integers(-3, 4, size=(2048, 8))
    rng.random((2048, 8))
    rng.integers(-3, 4, size=(2048, 8))
    rng.integers(-2, 3, size=(2048, 8))
    rng.standard_normal((512, 8))
    out = {}
    for b in (3, 4, 5):
        a = np.float32(O.compute_scale(1.0, b))
        x = rng.standard_normal((6000, 8)).astype(np.float32)
        out[b] = (x / a).astype(np.float32)
        rng.integers(0, 256, size=(3000, b))
    return out
