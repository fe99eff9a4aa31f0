"""Variable-rate KV cache: per-layer, per-K/V bits per dimension
(API of reference allocation/eval_alloc.py:56-145 and :224-250).

VariableRateKVCache compresses layer l's keys at bits_schedule[l]['K'] and
its values at bits_schedule[l]['V'], each update as one chunk with its own
scales and rANS tables, exactly like CompressedKVCache at that rate.  K and V
of an update are compressed in one batched launch sequence even when their
rates differ (codec.encode_batch takes one rate per chunk).

The perplexity harness of the reference module (model loading, wikitext,
sliding windows) is not on the compressed-KV path and is not reproduced.
"""
from __future__ import annotations

from typing import Dict, List

from ..llm.compressed_kv_cache import CompressedKVCache

__all__ = ["VariableRateKVCache", "allocation_to_schedule", "schedule_avg", "schedule_summary", "cyclic_schedule"]


class VariableRateKVCache(CompressedKVCache):
    """CompressedKVCache with bits_schedule = [{'K': b, 'V': b}, ...], one dict per
    layer (reference allocation/eval_alloc.py:56-145).  Layers beyond the
    schedule use 4 bits for K and V, as the reference's fallback does (:89-93).

    Rates other than 3/4/5 are accepted, as in the reference (it bypasses the
    parent's check, :70-74); the scale formula sqrt(2 pi e sigma^2 4^-b) holds
    for any b."""

    def __init__(self, bits_schedule: List[Dict[str, int]], eval_only_no_entropy: bool = True):
        super().__init__(4, eval_only_no_entropy)
        for i, s in enumerate(bits_schedule):
            if not isinstance(s, dict) or "K" not in s or "V" not in s:
                raise ValueError(f"bits_schedule[{i}] must be a dict with 'K' and 'V'")
            for key in ("K", "V"):
                b = s[key]
                if int(b) != b or not 1 <= int(b) <= 8:
                    raise ValueError(f"bits_schedule[{i}][{key!r}] must be an integer rate in 1..8, got {b!r}")
        self.bits_schedule = [{"K": int(s["K"]), "V": int(s["V"])} for s in bits_schedule]

    def _layer_bits(self, layer_idx: int):
        if layer_idx < len(self.bits_schedule):
            s = self.bits_schedule[layer_idx]
        else:
            s = {"K": 4, "V": 4}
        # the reference leaves self.bits at the V rate of the last update (:104-106)
        self.bits = s["V"]
        return s["K"], s["V"]


def allocation_to_schedule(alloc: dict) -> List[Dict[str, int]]:
    """Allocator output (results/allocation_*.json: layers[].b_K_disc / b_V_disc,
    else rounded b_K / b_V) -> bits_schedule (reference allocation/eval_alloc.py:227-235)."""
    schedule = []
    for lr in alloc["layers"]:
        schedule.append({"K": int(lr.get("b_K_disc", round(lr["b_K"]))),
                         "V": int(lr.get("b_V_disc", round(lr["b_V"])))})
    return schedule


def schedule_avg(schedule: List[Dict[str, int]]) -> float:
    """Mean bits per dimension over K and V of every layer (reference :238-242)."""
    k = sum(s["K"] for s in schedule)
    v = sum(s["V"] for s in schedule)
    return (k + v) / (2 * len(schedule))


def schedule_summary(schedule: List[Dict[str, int]]) -> str:
    """One-line histogram of the K and V rates."""
    from collections import Counter
    ck = Counter(s["K"] for s in schedule)
    cv = Counter(s["V"] for s in schedule)
    fk = " ".join(f"{b}b:{n}" for b, n in sorted(ck.items()))
    fv = " ".join(f"{b}b:{n}" for b, n in sorted(cv.items()))
    return f"K [{fk}]  V [{fv}]  avg {schedule_avg(schedule):.3f} b/d over {len(schedule)} layers"


def cyclic_schedule(n_layers: int, seed: int, rates=(3, 4, 5)) -> List[Dict[str, int]]:
    """Seeded schedule cycling through `rates`: layer l gets rates[(l + s) % len(rates)]
    for K and V, s = seed % len(rates).  The layer-wise allocation workload
    (28 layers cycling 3/4/5 bits) uses it."""
    s = seed % len(rates)
    return [{"K": rates[(l + s) % len(rates)], "V": rates[(l + s) % len(rates)]} for l in range(n_layers)]
