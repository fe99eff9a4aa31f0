"""Host-side logic of the device wrappers that needs no GPU: the error word
that a look-back launch leaves beside its totals."""
import pytest
import torch

from latticequant_amd import codec


def test_compact_counts_reads_totals_cpu():
    assert codec.compact_counts(torch.tensor([5, 3, 0], dtype=torch.int64)) == (5, 3)


def test_compact_counts_raises_on_lookback_error_cpu():
    with pytest.raises(codec.LookbackError):
        codec.compact_counts(torch.tensor([5, 3, 1], dtype=torch.int64))


class _Pend:
    """A stand-in for codec.PendingEncode: untracked, never ready."""

    def __init__(self, nbytes):
        self.tracked = False
        self.nbytes = nbytes

    def ready(self):
        return False

    def retained_bytes(self):
        return self.nbytes


def _settled(monkeypatch, pends):
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache
    calls = []
    monkeypatch.setattr(codec, "settle_many", lambda ps: calls.append(list(ps)))
    c = CompressedKVCache(bits_per_dim=4)
    c._pending = [(p, []) for p in pends]
    c._settle_ready()
    return calls


def test_pending_small_batches_settle_by_count_cpu(monkeypatch):
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache
    n = CompressedKVCache.SETTLE_SMALL_COUNT
    assert _settled(monkeypatch, [_Pend(1024) for _ in range(n - 1)]) == []
    calls = _settled(monkeypatch, [_Pend(1024) for _ in range(n)])
    assert len(calls) == 1 and len(calls[0]) == n


def test_pending_small_batches_settle_by_bytes_cpu(monkeypatch):
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache
    cap = CompressedKVCache.SETTLE_SMALL_BYTES
    assert _settled(monkeypatch, [_Pend(cap // 4), _Pend(cap // 4)]) == []
    calls = _settled(monkeypatch, [_Pend(cap // 2), _Pend(cap // 2)])
    assert len(calls) == 1 and len(calls[0]) == 2
