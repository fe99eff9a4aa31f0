"""GPU parity of the public module-level entry points that stand in for the
reference's modules (latticequant_amd.core.*, latticequant_amd.llm.*),
called exactly as the reference's callers call them (not through the fused
chunk kernels):

* core.e8_quantizer.quantize_e8 (core/e8_quantizer.py:90-110):
  Q_E8(x / scale) * scale in fp32, against the oracle's encode_e8 (pinned by
  the reference-written e8.npz) at the reference's own scales.
* core.entropy_coder.e8_to_symbols / symbols_to_e8 (core/entropy_coder.py:46-89):
  bit-exact with the reference-written coset / free / c8h / back arrays of
  e8.npz, including dyadic ties, near ties, half-integers and signed zeros.
* llm.compressed_kv_cache.pack_coset_bits / unpack_coset_bits
  (llm/compressed_kv_cache.py:46-63): the golden chunk's coset_packed bytes
  from its coset bits, and back; ragged lengths against the oracle.
* CompressedKVCache._free_layer (llm/compressed_kv_cache.py:334-340): the
  layer's decompressed K / V become the (1, 1, 0, 1) placeholder of the model
  dtype, the compressed chunks and their accounting stay, other layers are
  untouched, and the freed layer's chunks still decode (the reference frees
  buffers for memory measurement only).
* core.compact_storage.check_representable on the replayed inputs of the
  reference's inrange{b} masks (core/compact_storage.py:235-249).
"""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
pytestmark = pytest.mark.gpu


def test_quantize_e8_wrapper_gpu():
    from latticequant_amd.core.e8_quantizer import quantize_e8
    g = np.load(os.path.join(G, "e8.npz"))
    rng = np.random.default_rng(41)
    for scale in g["scales"][:6]:
        s32 = np.float32(scale)
        x = (rng.standard_normal((3, 5, 64, 8)) * 2.0).astype(np.float32)   # any (..., 8) shape
        got = quantize_e8(torch.from_numpy(x).cuda(), float(scale))
        assert got.shape == x.shape and got.dtype == torch.float32
        want = (O.encode_e8((x.reshape(-1, 8) / s32).astype(np.float32)) * s32).astype(np.float32)
        np.testing.assert_array_equal(got.cpu().numpy().reshape(-1, 8), want)
    # CPU input comes back on the CPU
    x = torch.from_numpy(g["x"][:512])
    got = quantize_e8(x, 0.75)
    assert got.device.type == "cpu"
    want = (O.encode_e8((g["x"][:512] / np.float32(0.75)).astype(np.float32)) * np.float32(0.75)).astype(np.float32)
    np.testing.assert_array_equal(got.numpy(), want)


def test_e8_symbols_wrappers_golden_gpu():
    from latticequant_amd.core.entropy_coder import e8_to_symbols, symbols_to_e8
    g = np.load(os.path.join(G, "e8.npz"))
    coset, free, c8h = e8_to_symbols(torch.from_numpy(g["e8"]).cuda())
    assert coset.dtype == free.dtype == c8h.dtype == torch.int64
    np.testing.assert_array_equal(coset.cpu().numpy(), g["coset"])
    np.testing.assert_array_equal(free.cpu().numpy(), g["free"])
    np.testing.assert_array_equal(c8h.cpu().numpy(), g["c8h"])
    back = symbols_to_e8(torch.from_numpy(g["coset"]).cuda(), torch.from_numpy(g["free"]).cuda(),
                         torch.from_numpy(g["c8h"]).cuda())
    np.testing.assert_array_equal(back.cpu().numpy(), g["back"])
    np.testing.assert_array_equal(back.cpu().numpy(), g["e8"])   # lossless
    # the D8 points (coset 0 only) through the same pair, from CPU tensors
    c2, f2, h2 = e8_to_symbols(torch.from_numpy(g["d8"]))
    assert c2.device.type == "cpu" and int(c2.sum()) == 0
    oc, of, oh = O.e8_to_symbols(g["d8"])
    np.testing.assert_array_equal(f2.numpy(), of)
    np.testing.assert_array_equal(h2.numpy(), oh)
    np.testing.assert_array_equal(symbols_to_e8(c2, f2, h2).numpy(), g["d8"])


def test_coset_bit_packing_wrappers_gpu():
    from latticequant_amd.llm.compressed_kv_cache import pack_coset_bits, unpack_coset_bits
    g = np.load(os.path.join(G, "cache.npz"))
    for ci in range(int(g["n_cases"])):
        p = f"c{ci}_"
        packed = g[p + "coset_packed"]
        n = int(np.asarray(g[p + "coset_counts"]).sum())
        bits = O.unpack_coset_bits(packed, n)
        got = pack_coset_bits(torch.from_numpy(bits.astype(np.int64)).cuda())
        np.testing.assert_array_equal(got.cpu().numpy(), packed)
        back = unpack_coset_bits(torch.from_numpy(packed).cuda(), n)
        np.testing.assert_array_equal(back.cpu().numpy(), bits)
    rng = np.random.default_rng(5)
    for n in (0, 1, 7, 8, 9, 63, 64, 65, 1000, 4099):
        bits = (rng.random(n) < 0.5).astype(np.uint8)
        got = pack_coset_bits(torch.from_numpy(bits))   # CPU in, CPU out
        assert got.device.type == "cpu"
        np.testing.assert_array_equal(got.numpy(), O.pack_coset_bits(bits))
        np.testing.assert_array_equal(unpack_coset_bits(got.cuda(), n).cpu().numpy(), bits)
    with pytest.raises(ValueError):
        unpack_coset_bits(torch.zeros(1, dtype=torch.uint8).cuda(), 9)


def test_free_layer_gpu():
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache
    gen = torch.Generator().manual_seed(17)
    cache = CompressedKVCache(bits_per_dim=4)
    xs = {l: torch.randn(1, 4, 24, 128, generator=gen).half().cuda() for l in range(2)}
    for l, x in xs.items():
        cache.update(x, x, l)
    before = cache.compressed_bytes()
    kept_k = cache.key_cache[1].clone()
    cache._free_layer(0)
    for t in (cache.key_cache[0], cache.value_cache[0]):
        assert t.shape == (1, 1, 0, 1) and t.dtype == torch.float16 and t.device.type == "cuda"
    assert torch.equal(cache.key_cache[1], kept_k)
    assert cache.compressed_bytes() == before
    assert len(cache._comp_keys[0].chunks) == 1 and cache.get_seq_length(0) == 24
    cache._free_layer(5)   # past the last layer: no-op, as in the reference
    # the freed layer's chunks still decode to what update() returned
    ch = cache._comp_keys[0].chunks[0]
    s32 = ch.encoded.scale32.cpu().numpy()
    ref = O.compress_chunk(xs[0].cpu().numpy(), 4, scales_f32=s32)
    np.testing.assert_array_equal(cache._decompress_chunk(ch).cpu().numpy(), O.decompress_chunk(ref))


def test_check_representable_inrange_fixture_gpu():
    """core.compact_storage.check_representable on the replayed compact.npz
    inputs equals the reference's inrange{b} masks (rejections included)."""
    from latticequant_amd.core import compact_storage as cs
    from tests.golden.replay import compact_inputs
    g = np.load(os.path.join(G, "compact.npz"))
    for b, x in compact_inputs().items():
        q = O.encode_e8(x)
        got = cs.check_representable(torch.from_numpy(q).cuda(), b).cpu().numpy()
        np.testing.assert_array_equal(got, g[f"inrange{b}"])


def test_deferred_entropy_coding_equals_per_update_gpu():
    """Small updates (decode steps) quantize at once and entropy-code in shared
    groups: the K / V update() returns and every chunk's words, streams, byte
    counts and decoded tensor equal those of a cache that encodes each update
    on its own, over a prefill plus decode steps of three layers with a group
    limit small enough to flush several groups; a chunk of a group that is
    still open is read (and settled) mid-run; one chunk against the oracle."""
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache
    gen = torch.Generator().manual_seed(29)
    a = CompressedKVCache(bits_per_dim=4)
    a.DEFER_CHUNKS = 8
    b = CompressedKVCache(bits_per_dim=4)
    b.DEFER_MAX_VECTORS = 0
    layers, heads = 3, 2
    xs = {}
    for step in range(12):
        T = 40 if step == 0 else 1
        for l in range(layers):
            k = torch.randn(1, heads, T, 128, generator=gen)
            k[..., :3] *= 6.0
            k = k.half().cuda()
            v = torch.randn(1, heads, T, 128, generator=gen).half().cuda()
            xs[(step, l)] = k
            ka, va = a.update(k, v, l)
            kb, vb = b.update(k, v, l)
            assert torch.equal(ka, kb) and torch.equal(va, vb)
        if step == 5:   # read a chunk of the open group: it is encoded and settled now
            assert a._comp_keys[0].chunks[-1].reference_bytes() == b._comp_keys[0].chunks[-1].reference_bytes()
    assert a.compressed_bytes() == b.compressed_bytes()
    for l in range(layers):
        for ca, cb in zip(a._comp_keys[l].chunks + a._comp_values[l].chunks,
                          b._comp_keys[l].chunks + b._comp_values[l].chunks):
            assert torch.equal(ca.gpu_bitstream, cb.gpu_bitstream)
            assert torch.equal(ca.coset_packed, cb.coset_packed)
            assert ca.side_info_bytes() == cb.side_info_bytes()
            assert [s.n_bits for s in ca.streams] == [s.n_bits for s in cb.streams]
            assert torch.equal(a._decompress_chunk(ca), b._decompress_chunk(cb))
    ch = a._comp_keys[1].chunks[7]   # layer 1, decode step 7
    s32 = ch.encoded.scale32.cpu().numpy()
    ref = O.compress_chunk(xs[(7, 1)].cpu().numpy(), 4, scales_f32=s32)
    np.testing.assert_array_equal(ch.gpu_bitstream.cpu().numpy().view(np.uint32), ref.bitstream.astype(np.uint32))
