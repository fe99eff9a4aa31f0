"""Allocator feed of the variable-rate cache (reference allocation/allocator.py),
CPU only.  discretise is pinned by the reference's published schedule: its
continuous rates and greedy integer rates for Qwen2.5-7B at 4 b/d; slots
strictly inside (3, 5) are unclamped, so their weights are 2^(2 b) up to one
common factor, which leaves the upgrade order unchanged, and clamped slots sit
on allowed rates (no upgrade).  water_filling is pinned by its closed form,
the budget, the bounds and the common water level of the free slots."""
import json
import os

import numpy as np
import pytest

from latticequant_amd.allocation.allocator import allocate, compute_weights, discretise, water_filling
from latticequant_amd.allocation.eval_alloc import allocation_to_schedule

GOLD = os.path.join(os.path.dirname(__file__), "golden", "allocation_Qwen2.5-7B_4b.json")


def test_discretise_reproduces_published_schedule():
    g = json.load(open(GOLD))
    b = np.array([[lr["b_K"], lr["b_V"]] for lr in g["layers"]])
    want = np.array([[lr["b_K_disc"], lr["b_V_disc"]] for lr in g["layers"]])
    w = 2.0 ** (2.0 * b)
    got = discretise(b, w, 4.0)
    np.testing.assert_array_equal(got, want)
    assert got.mean() == g["budget_discrete"]


def test_discretise_weight_order_matters():
    # two slots at 3.5 with a budget for one upgrade: the heavier weight wins
    b = np.array([[3.5, 3.5]])
    assert discretise(b, np.array([[1.0, 2.0]]), 4.0 - 0.5).tolist() == [[3, 4]]
    assert discretise(b, np.array([[2.0, 1.0]]), 4.0 - 0.5).tolist() == [[4, 3]]


def test_water_filling_unclamped_closed_form():
    rng = np.random.default_rng(0)
    w = rng.lognormal(0.0, 1.0, size=(28, 2))
    r = water_filling(w, budget=4.0, b_min=-100, b_max=100)
    lw = np.log2(w)
    np.testing.assert_allclose(r["bits"], 4.0 + 0.5 * (lw - lw.mean()), rtol=0, atol=1e-12)
    assert r["n_iter"] == 1
    np.testing.assert_allclose(r["gain"], w.mean() / np.exp(np.log(w).mean()), rtol=1e-12)


@pytest.mark.parametrize("seed", range(5))
def test_water_filling_clamped_invariants(seed):
    rng = np.random.default_rng(seed)
    w = rng.lognormal(0.0, 3.0, size=(32, 2))
    r = water_filling(w, budget=4.0, b_min=3.0, b_max=5.0)
    b = r["bits"].reshape(-1)
    assert (b >= 3.0).all() and (b <= 5.0).all()
    np.testing.assert_allclose(b.mean(), 4.0, atol=1e-12)
    free = (b > 3.0) & (b < 5.0)
    lvl = b[free] - 0.5 * np.log2(w.reshape(-1)[free])
    np.testing.assert_allclose(lvl, lvl[0], atol=1e-12)   # one water level
    # a clamped-high slot is at least as heavy as every free one, a clamped-low one no heavier
    wf = w.reshape(-1)
    if (b == 5.0).any() and free.any():
        assert wf[b == 5.0].min() >= wf[free].max()
    if (b == 3.0).any() and free.any():
        assert wf[b == 3.0].max() <= wf[free].min()


def test_allocate_record_feeds_the_cache_schedule():
    sens = {"model": "toy", "layers": [{"eta_K": 1.0 + l, "sigma2_K": 2.0, "eta_V": 1.0, "sigma2_V": 1.0 + 0.5 * l}
                                       for l in range(6)]}
    prop = {"layers": [{"gamma": 1.0 + 0.1 * l} for l in range(6)]}
    w = compute_weights(sens, prop)
    np.testing.assert_allclose(w[3], [(1 + 3) * 2.0 * 1.3, 1.0 * 2.5 * 1.3])
    out = allocate(sens, prop, budget=4.0, b_min=3.0, b_max=5.0, discrete=True)
    sched = allocation_to_schedule(out)
    assert len(sched) == 6 and all(s["K"] in (3, 4, 5) and s["V"] in (3, 4, 5) for s in sched)
    assert out["budget_discrete"] == np.mean([[s["K"], s["V"]] for s in sched])
    with pytest.raises(ValueError):
        compute_weights(sens, {"layers": prop["layers"][:5]})
