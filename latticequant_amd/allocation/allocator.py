"""Per-layer K/V bit allocation that feeds VariableRateKVCache (host code).

The reference computes a schedule once, offline, on the CPU
(allocation/allocator.py); the cache then consumes it through
``allocation_to_schedule``.  This module is that producer, so that a
sensitivity file can be turned into a schedule without the reference:

    weights    w[l, X] = gamma_l * eta_X,l * sigma2_X,l      (:61-99)
    continuous b = mean budget + 1/2 log2(w / GM(w)), clamped to
               [b_min, b_max] with the budget redistributed over the free
               slots until no slot leaves the bounds            (:106-194)
    discrete   every slot snapped down to an allowed rate, then upgraded in
               descending order of the distortion it removes,
               w (2^-2 floor - 2^-2 ceil), while budget is left  (:197-270)

The iteration order of the clamping loop and the upgrade order (numpy's
default argsort of the negated gains) decide the result on ties, so they
follow the reference's steps; the arithmetic is vectorised numpy.
"""
from __future__ import annotations

import json
import warnings
from typing import Optional, Sequence

import numpy as np


def compute_weights(sensitivity: dict, propagation: Optional[dict] = None) -> np.ndarray:
    """(n_layers, 2) effective weights [w_K, w_V] (reference allocator.py:61-99).
    A layer may give w_K / w_V directly, else eta * sigma2; gamma defaults to 1."""
    layers = sensitivity["layers"]
    n = len(layers)
    if propagation is not None:
        if len(propagation["layers"]) != n:
            raise ValueError(f"Layer count mismatch: sensitivity has {n} layers "
                             f"but propagation has {len(propagation['layers'])}.")
        gamma = np.array([float(p["gamma"]) for p in propagation["layers"]])
    else:
        gamma = np.ones(n)
    w = np.array([[lr["w_K"] if "w_K" in lr else lr["eta_K"] * lr["sigma2_K"],
                   lr["w_V"] if "w_V" in lr else lr["eta_V"] * lr["sigma2_V"]] for lr in layers], dtype=np.float64)
    return w * gamma[:, None]


def water_filling(weights: np.ndarray, budget: float = 4.0, b_min: float = 2.0, b_max: float = 8.0,
                  max_iter: int = 20) -> dict:
    """Clamped continuous allocation (reference allocator.py:106-194).
    Returns bits (n_layers, 2), gain = AM(w) / GM(w), budget_actual, n_iter."""
    w = np.asarray(weights, dtype=np.float64).reshape(-1)
    n_layers = np.asarray(weights).shape[0]
    ok = w > 0
    if not ok.all():
        warnings.warn(f"{int((~ok).sum())} of {w.size} weight(s) are <= 0; using the smallest positive weight")
        w = np.where(ok, w, w[ok].min() if ok.any() else 1e-30)
    lw = np.log2(w)
    gain = float(w.mean() / 2.0 ** lw.mean())
    bits = np.full(w.size, float(budget))
    fixed = np.zeros(w.size, dtype=bool)
    it = 0
    for it in range(max_iter):
        free = np.flatnonzero(~fixed)
        if free.size == 0:
            break
        spare = budget * w.size - (bits[fixed].sum() if fixed.any() else 0.0)
        lf = lw[free]
        # same association as the reference, so the bits agree to the last ulp
        b = spare / free.size + 0.5 * (lf - np.log2(2.0 ** lf.mean()))
        lo, hi = b < b_min, b > b_max
        b[lo] = b_min
        b[hi] = b_max
        bits[free] = b
        hit = lo | hi
        fixed[free[hit]] = True
        if not hit.any():
            break
    return {"bits": bits.reshape(n_layers, 2), "gain": gain, "budget_actual": float(bits.mean()),
            "n_iter": it + 1}


def discretise(bits_continuous: np.ndarray, weights: np.ndarray, budget: float,
               allowed: Sequence[int] = (3, 4, 5)) -> np.ndarray:
    """Objective-aware greedy rounding to allowed integer rates
    (reference allocator.py:197-270)."""
    shape = np.asarray(bits_continuous).shape
    b = np.asarray(bits_continuous, dtype=np.float64).reshape(-1)
    w = np.asarray(weights, dtype=np.float64).reshape(-1)
    al = np.array(sorted(allowed))
    # largest allowed <= b (else the smallest), smallest allowed >= b (else the largest)
    fl = al[np.clip(np.searchsorted(al, b, side="right") - 1, 0, al.size - 1)]
    ce = al[np.clip(np.searchsorted(al, b, side="left"), 0, al.size - 1)]
    step = ce - fl
    gain = np.where(step > 0, w * (2.0 ** (-2.0 * fl) - 2.0 ** (-2.0 * ce)), 0.0)
    out = fl.copy()
    left = budget * b.size - fl.sum()
    for i in np.argsort(-gain):
        if left <= 0:
            break
        if 0 < step[i] <= left + 0.5:
            out[i] = ce[i]
            left -= step[i]
    return out.reshape(shape)


def allocate(sensitivity, propagation=None, budget: float = 4.0, b_min: float = 2.0, b_max: float = 8.0,
             discrete: bool = False, allowed_bits: Sequence[int] = (3, 4, 5)) -> dict:
    """Sensitivity (dict or JSON path) [+ propagation] -> the allocation record
    the reference writes (allocator.py:276-345): per layer w_K, w_V, b_K, b_V
    and, with discrete=True, b_K_disc / b_V_disc.  allocation_to_schedule
    turns it into the cache's bits schedule."""
    prop_src = propagation if isinstance(propagation, str) else None
    if isinstance(sensitivity, str):
        with open(sensitivity) as f:
            sensitivity = json.load(f)
    if isinstance(propagation, str):
        with open(propagation) as f:
            propagation = json.load(f)
    w = compute_weights(sensitivity, propagation)
    r = water_filling(w, budget=budget, b_min=b_min, b_max=b_max)
    out = {"model": sensitivity.get("model", "unknown"), "n_layers": len(sensitivity["layers"]),
           "uniform_budget": budget,
           "gamma_source": prop_src if prop_src else ("given" if propagation is not None else "default (Γ=1)"),
           "gain_am_gm": r["gain"], "budget_actual": r["budget_actual"], "n_iter": r["n_iter"],
           "b_min": b_min, "b_max": b_max,
           "layers": [{"layer": l, "w_K": float(w[l, 0]), "w_V": float(w[l, 1]),
                       "b_K": float(r["bits"][l, 0]), "b_V": float(r["bits"][l, 1])} for l in range(w.shape[0])]}
    if discrete:
        d = discretise(r["bits"], w, budget, allowed=allowed_bits)
        for l, e in enumerate(out["layers"]):
            e["b_K_disc"], e["b_V_disc"] = int(d[l, 0]), int(d[l, 1])
        out["budget_discrete"] = float(d.mean())
        out["discrete_method"] = "objective_aware_greedy"
        out["allowed_bits"] = list(allowed_bits)
    return out
