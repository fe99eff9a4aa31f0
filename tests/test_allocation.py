"""Variable-rate cache (reference allocation/eval_alloc.py:56-145, :224-250).

CPU: the schedule helpers on the reference's published Qwen2.5-7B 4-bit
allocation (tests/golden/allocation_Qwen2.5-7B_4b.json, data of the reference).
GPU: every layer's K and V chunks of a VariableRateKVCache equal the oracle's
compress_chunk at that layer's K / V rate, bit for bit."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _alloc():
    with open(os.path.join(G, "allocation_Qwen2.5-7B_4b.json")) as f:
        return json.load(f)


def test_allocation_to_schedule_reference_file():
    from latticequant_amd.allocation.eval_alloc import allocation_to_schedule, schedule_avg, schedule_summary
    a = _alloc()
    s = allocation_to_schedule(a)
    assert len(s) == a["n_layers"] == 28
    assert [x["K"] for x in s] == [lr["b_K_disc"] for lr in a["layers"]]
    assert [x["V"] for x in s] == [lr["b_V_disc"] for lr in a["layers"]]
    assert schedule_avg(s) == pytest.approx(a["budget_discrete"])
    # without the discrete fields the continuous rates are rounded
    s2 = allocation_to_schedule({"layers": [{"b_K": 3.4, "b_V": 4.6}, {"b_K": 5.0, "b_V": 2.5}]})
    assert s2 == [{"K": 3, "V": 5}, {"K": 5, "V": 2}]
    assert "avg 4.000" in schedule_summary(s)


def test_cyclic_schedule_and_validation():
    from latticequant_amd.allocation.eval_alloc import VariableRateKVCache, cyclic_schedule
    s = cyclic_schedule(28, seed=7)
    assert [x["K"] for x in s[:4]] == [4, 5, 3, 4] and all(x["K"] == x["V"] for x in s)
    with pytest.raises(ValueError):
        VariableRateKVCache([{"K": 4}])
    with pytest.raises(ValueError):
        VariableRateKVCache([{"K": 4.5, "V": 4}])


@pytest.mark.gpu
def test_variable_rate_cache_vs_oracle_gpu():
    from latticequant_amd.allocation.eval_alloc import VariableRateKVCache
    sched = [{"K": 3, "V": 5}, {"K": 5, "V": 3}, {"K": 4, "V": 4}]
    cache = VariableRateKVCache(sched, eval_only_no_entropy=False)
    gen = torch.Generator().manual_seed(31)
    inputs = {}
    for T in (24, 1, 3):
        for layer in range(4):   # layer 3 is beyond the schedule: 4 / 4 bits
            k = torch.randn(1, 4, T, 64, generator=gen).half()
            v = torch.randn(1, 4, T, 64, generator=gen).half()
            cache.update(k.cuda(), v.cuda(), layer)
            inputs.setdefault(layer, []).append((k, v))
    assert cache.get_seq_length(0) == 28
    for layer in range(4):
        bk, bv = (sched[layer]["K"], sched[layer]["V"]) if layer < 3 else (4, 4)
        for (k, v), ck, cv in zip(inputs[layer], cache._comp_keys[layer].chunks, cache._comp_values[layer].chunks):
            for t, ch, b in ((k, ck, bk), (v, cv, bv)):
                assert ch.bits_per_dim == b
                ref = O.compress_chunk(t.numpy(), b, scales_f32=ch.encoded.scale32.cpu().numpy())
                np.testing.assert_array_equal(ch.gpu_bitstream.cpu().numpy().view(np.uint32), ref.bitstream)
                np.testing.assert_array_equal(cache._decompress_chunk(ch).cpu().numpy(), O.decompress_chunk(ref))
                # scale formula at the chunk's own rate
                s2 = ch.encoded.sigma2.cpu().numpy()
                np.testing.assert_allclose(ch.encoded.scale32.cpu().numpy(),
                                           np.sqrt(2 * np.pi * np.e * s2 * 4.0 ** (-b)), rtol=1e-6)
