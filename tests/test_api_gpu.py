"""GPU parity of the reference-API modules (latticequant_amd.core.*, .llm.*)
against the CPU oracle and the reference's golden vectors (tests/golden).

Integer / byte outputs are compared bit-exactly; fp16 outputs too (the
contract allows 1 ulp, the kernels reproduce the reference's rounding)."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
pytestmark = pytest.mark.gpu


def _ragged(g, key, i):
    off = g[key + "_off"]
    return g[key][off[i]:off[i + 1]]


# ------------------------------------------------------------------- rANS --

def test_build_rans_table_golden_gpu():
    from latticequant_amd.core import gpu_ans as ga
    g = np.load(os.path.join(G, "rans.npz"))
    n = len(g["tab_lo"])
    counts = [_ragged(g, "tab_counts", i) for i in range(n)]
    alph = [list(range(int(g["tab_lo"][i]), int(g["tab_lo"][i]) + len(counts[i]))) for i in range(n)]
    tabs = ga.build_rans_tables(counts, alph)
    wide = 0
    for i, t in enumerate(tabs):
        assert t.cumfreqs[0] == 0 and t.cumfreqs[-1] == ga.L and (t.freqs >= 1).all()
        assert t.status == 0, f"table {i}"
        np.testing.assert_array_equal(t.freqs, g["tab_freqs"][g["tab_counts_off"][i]:g["tab_counts_off"][i + 1]],
                                      err_msg=f"table {i}")
        np.testing.assert_array_equal(t.lookup, g["tab_lookup"][i])
        wide += t.n_symbols > 256
    assert wide > 0   # the golden set holds alphabets above 256 symbols (numpy's quicksort order)
    # single-table API
    t = ga.build_rans_table(counts[0], alph[0])
    np.testing.assert_array_equal(t.freqs, tabs[0].freqs)


def test_rans_encode_golden_gpu():
    from latticequant_amd.core import gpu_ans as ga
    g = np.load(os.path.join(G, "rans.npz"))
    n = len(g["enc_lo"])
    syms = [_ragged(g, "enc_syms", i) for i in range(n)]
    counts = [_ragged(g, "enc_counts", i) for i in range(n)]
    alph = [list(range(int(g["enc_lo"][i]), int(g["enc_lo"][i]) + len(counts[i]))) for i in range(n)]
    tabs = ga.build_rans_tables(counts, alph)
    res = ga.rans_encode_many(syms, tabs)
    for i, (w, st, nb) in enumerate(res):
        np.testing.assert_array_equal(w, _ragged(g, "enc_words", i), err_msg=f"stream {i}")
        assert st == g["enc_state"][i] and nb == g["enc_nbits"][i]
    # the reference's GPU decoder semantics (test_gpu_vs_cpu, core/gpu_ans.py:468-510)
    streams = [ga.RANSStream(bitstream=w, n_bits=nb, initial_state=st, n_symbols=len(s), table=t)
               for (w, st, nb), s, t in zip(res, syms, tabs)]
    dec = ga.gpu_rans_decode(streams)
    for i, d in enumerate(dec):
        np.testing.assert_array_equal(d, syms[i])
    np.testing.assert_array_equal(ga.rans_decode_cpu(res[0][0], res[0][2], res[0][1], tabs[0], len(syms[0])), syms[0])


def test_rans_reference_distributions_gpu():
    """core/gpu_ans.py:382-424 count vectors, seed 42; GPU encode == oracle, decode round trip."""
    from latticequant_amd.core import gpu_ans as ga
    rng = np.random.default_rng(42)
    cases = [(list(range(-5, 6)), [1, 3, 10, 30, 50, 60, 50, 30, 10, 3, 1]),
             (list(range(5)), [500, 10, 3, 2, 1]), (list(range(8)), [13, 12, 13, 12, 13, 12, 13, 12]),
             ([0, 1], [70, 30]), (list(range(-3, 4)), [1, 1, 1, 200, 1, 1, 1]),
             (list(range(-40, 41)), list(np.exp(-np.arange(-40, 41) ** 2 / 200.0) * 1e4 + 1)),
             ([7], [5])]
    for alph, counts in cases:
        counts = np.asarray(counts).astype(np.int64)
        t = ga.build_rans_table(counts, alph)
        to = O.build_rans_table(counts, alph)
        np.testing.assert_array_equal(t.freqs, to.freqs)
        s = rng.choice(alph, size=3000, p=counts / counts.sum())
        w, st, nb = ga.rans_encode(s, t)
        wo, sto, nbo = O.rans_encode(s, to)
        np.testing.assert_array_equal(w, wo)
        assert (st, nb) == (sto, nbo)
        np.testing.assert_array_equal(ga.rans_decode_cpu(w, nb, st, t, len(s)), s)


def test_rans_symbol_lookup_rules_gpu():
    """Out-of-alphabet symbols take the nearest entry (first on ties); duplicate
    alphabet values resolve to the last index (core/gpu_ans.py:110-119)."""
    from latticequant_amd.core import gpu_ans as ga
    alph = [5, -3, 0, 9, 0]
    counts = np.array([4, 7, 9, 2, 3], np.int64)
    t = ga.build_rans_table(counts, alph)
    to = O.build_rans_table(counts, alph)
    s = np.array([5, -3, 0, 9, 1, 2, 100, -100, 7, -2, 4, 3])
    w, st, nb = ga.rans_encode(s, t)
    wo, sto, nbo = O.rans_encode(s, to)
    np.testing.assert_array_equal(w, wo)
    assert (st, nb) == (sto, nbo)
    # contiguous alphabet, symbols beyond both ends
    t2 = ga.build_rans_table(np.array([3, 5, 2], np.int64), [0, 1, 2])
    w, st, nb = ga.rans_encode(np.array([-7, 9, 1]), t2)
    np.testing.assert_array_equal(ga.rans_decode_cpu(w, nb, st, t2, 3), [0, 2, 1])
    w, st, nb = ga.rans_encode(np.zeros(0, np.int64), t2)
    assert (st, nb, w.tolist()) == (1024, 0, [0])


def test_rans_alphabet_limit_gpu():
    from latticequant_amd.core import gpu_ans as ga
    with pytest.raises(ValueError):
        ga.build_rans_table(np.ones(1025, np.int64), list(range(1025)))


# ---------------------------------------------------------- compact form --

def test_compact_golden_gpu():
    from latticequant_amd.core import compact_storage as cs
    g = np.load(os.path.join(G, "compact.npz"))
    for b in (3, 4, 5):
        p = cs.pack_e8(torch.from_numpy(g[f"q{b}"]).cuda(), b)
        np.testing.assert_array_equal(p.cpu().numpy(), g[f"packed{b}"])
        u = cs.unpack_e8(torch.from_numpy(g[f"raw{b}"]).cuda(), b)
        np.testing.assert_array_equal(u.cpu().numpy(), g[f"unpacked{b}"])


def test_validate_and_representable_gpu():
    from latticequant_amd.core import compact_storage as cs
    g = np.load(os.path.join(G, "e8.npz"))
    q = np.concatenate([g["e8"], g["x"][:4096]])          # valid points, then mostly invalid ones
    v, c = cs.validate_e8(torch.from_numpy(q).cuda())
    vo, co = O.validate_e8(q)
    np.testing.assert_array_equal(v.cpu().numpy(), vo)
    np.testing.assert_array_equal(c.cpu().numpy(), co)
    for b in (3, 4, 5):
        np.testing.assert_array_equal(cs.check_representable(torch.from_numpy(q).cuda(), b).cpu().numpy(),
                                      O.check_representable(q, b))
    for bad in ([1.0, 0, 0, 0, 0, 0, 0, 0], [1.0, 0.5, 0, 0, 0, 0, 0, 0], [8.0, 8.0, 0, 0, 0, 0, 0, 0]):
        with pytest.raises(ValueError):
            cs.pack_e8(torch.tensor([bad]).cuda(), 4)


def test_triton_unpack_4bit_gpu(monkeypatch):
    from latticequant_amd.core import triton_dequant as td
    rng = np.random.default_rng(3)
    n, H = 50000, 8
    q = O.encode_e8(rng.standard_normal((n, 8)).astype(np.float32) * 2.5)
    ok = O.check_representable(q, 4)
    q = q[ok]
    packed = O.pack_e8(q, 4)
    head = rng.integers(0, H, size=len(q)).astype(np.int32)
    scales = (rng.random(H) + 0.1).astype(np.float32)
    out = td.triton_unpack_e8_4bit(torch.from_numpy(packed).cuda(), torch.from_numpy(scales).cuda(),
                                   torch.from_numpy(head).cuda())
    np.testing.assert_array_equal(out.cpu().numpy(), O.dequant_compact(packed, 4, scales, head))
    monkeypatch.setenv("LQ_DEBUG_CHECKS", "1")   # the host-side range check (a sync) is opt-in
    with pytest.raises(ValueError):
        td.triton_unpack_e8_4bit(torch.from_numpy(packed).cuda(), torch.from_numpy(scales).cuda(),
                                 torch.from_numpy(head + H).cuda())


# ------------------------------------------------------------------- RHT --

def test_rht_golden_gpu():
    from latticequant_amd.core import pipeline as pl
    g = np.load(os.path.join(G, "rht.npz"))
    for s, sg in zip(g["seeds"], g["signs"]):
        np.testing.assert_array_equal(pl.RHT(128, seed=int(s)).signs.numpy(), sg)
    r = pl.RHT(128, seed=7)
    y = r.forward(torch.from_numpy(g["x"]).cuda())
    np.testing.assert_array_equal(y.cpu().numpy(), g["y"])
    back = r.inverse(y)
    np.testing.assert_array_equal(back.cpu().numpy(), O.rht_f32(g["y"], g["signs"][2], inverse=True))
    # head-batched transform, every power-of-two width the kernel takes
    rng = np.random.default_rng(4)
    for d in (8, 16, 32, 64, 128, 256, 512):
        x = rng.standard_normal((2, 3, 5, d)).astype(np.float32)
        # rows that take the division's IEEE branch: zeros (their sign), tiny and huge values
        x[0, 0, 0] = 0.0
        x[0, 0, 1] = -0.0
        x[0, 1, 2] = 1e-33
        x[1, 2, 3, : d // 2] = 1.0e35   # large, and the sums stay finite
        x[1, 1, 4, 0] = -2.0 ** -120
        signs = pl.head_signs(d, 3, 3, 1)
        y = pl.rht_heads(torch.from_numpy(x).cuda(), signs)
        want = np.stack([O.rht_f32(x[:, h], signs[h].numpy()) for h in range(3)], 1)
        np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
        back = pl.rht_heads(y, signs, inverse=True)
        wantb = np.stack([O.rht_f32(want[:, h], signs[h].numpy(), inverse=True) for h in range(3)], 1)
        np.testing.assert_array_equal(back.cpu().numpy().view(np.uint32), wantb.view(np.uint32))
        x16 = torch.from_numpy(x).half()
        y16 = pl.rht_heads(x16.cuda(), signs, out_dtype=torch.float16)
        want16 = np.stack([O.rht_f32(x16[:, h].float().numpy(), signs[h].numpy()) for h in range(3)], 1)
        np.testing.assert_array_equal(y16.cpu().numpy(), want16.astype(np.float16))


# -------------------------------------------------------- KV cache (HF) --

def _chunk_fields_match(ch, g, p):
    np.testing.assert_array_equal(ch.gpu_bitstream.cpu().numpy().view(np.uint32), g[p + "bitstream"])
    np.testing.assert_array_equal(ch.coset_packed.cpu().numpy(), g[p + "coset_packed"])
    assert ch.coset_counts == tuple(int(v) for v in g[p + "coset_counts"])
    np.testing.assert_array_equal(np.array(ch.stream_word_offsets), g[p + "word_offsets"])
    np.testing.assert_array_equal(np.array(ch.stream_meta).reshape(-1, 3), g[p + "stream_meta"])
    np.testing.assert_array_equal([s.initial_state for s in ch.streams], g[p + "states"])
    np.testing.assert_array_equal([s.n_bits for s in ch.streams], g[p + "nbits"])
    np.testing.assert_array_equal([s.table.alphabet[0] for s in ch.streams], g[p + "alpha_lo"])
    np.testing.assert_array_equal(np.concatenate([s.table.freqs for s in ch.streams]), g[p + "freqs"])
    np.testing.assert_array_equal(ch.scales.cpu().numpy(), g[p + "scales"])
    assert ch.reference_bytes() == int(g[p + "compressed_bytes"])


def test_cache_update_golden_gpu():
    """One update() per golden case: the chunk and both dequant variants equal
    what the reference's CompressedKVCache wrote (tests/golden/cache.npz)."""
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache
    g = np.load(os.path.join(G, "cache.npz"))
    for ci in range(int(g["n_cases"])):
        p = f"c{ci}_"
        t = torch.from_numpy(g[p + "input"]).cuda()
        cache = CompressedKVCache(bits_per_dim=int(g[p + "bits"]))
        ch, dec = cache._compress_tensor(t)
        # the device computes sigma^2 in another summation order than torch's CPU mean;
        # the scales (fp16) are compared and must agree, then everything downstream is exact
        _chunk_fields_match(ch, g, p)
        np.testing.assert_array_equal(dec.cpu().numpy(), g[p + "decompressed"])
        np.testing.assert_array_equal(cache._decompress_chunk(ch).cpu().numpy(), g[p + "rebuilt"])
        k, v = cache.update(t, t, 0)
        np.testing.assert_array_equal(k.cpu().numpy(), g[p + "decompressed"])
        assert cache.get_seq_length(0) == t.shape[2]
        assert cache.compressed_bytes() == 2 * int(g[p + "compressed_bytes"])


def test_cache_incremental_decode_gpu():
    """Prefill + 1-token steps over 3 layers (llm/compressed_kv_cache.py:476-496, 570-596):
    returned K/V are the concatenated per-update dequantised tensors, every chunk
    matches the oracle's compress_chunk, and _decompress_chunk rebuilds q * scale16."""
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache
    gen = torch.Generator().manual_seed(9)
    cache = CompressedKVCache(bits_per_dim=4)
    hist = {l: ([], []) for l in range(3)}
    steps = [37] + [1] * 6 + [5]
    for T in steps:
        for layer in range(3):
            k = torch.randn(1, 8, T, 128, generator=gen).half()
            v = torch.randn(1, 8, T, 128, generator=gen).half()
            kf, vf = cache.update(k.cuda(), v.cuda(), layer)
            hist[layer][0].append(k)
            hist[layer][1].append(v)
            assert kf.shape == (1, 8, sum(steps[:len(hist[layer][0])]), 128)
            assert cache.get_mask_sizes(1, layer) == (kf.shape[2] + 1, 0)
    assert cache.get_seq_length(2) == sum(steps)
    for layer in range(3):
        want_k = []
        for ci, (k, ch) in enumerate(zip(hist[layer][0], cache._comp_keys[layer].chunks)):
            sc = ch.scales.float().cpu().numpy()
            ref = O.compress_chunk(k.numpy(), 4, scales_f32=None)
            # scales come from each device's own sigma^2: compare them, then run the oracle on ours
            np.testing.assert_allclose(sc, ref.scales.astype(np.float32), rtol=1e-3)
            s32 = ch.encoded.scale32.cpu().numpy()
            ref = O.compress_chunk(k.numpy(), 4, scales_f32=s32)
            np.testing.assert_array_equal(ch.gpu_bitstream.cpu().numpy().view(np.uint32), ref.bitstream)
            np.testing.assert_array_equal(cache._decompress_chunk(ch).cpu().numpy(), O.decompress_chunk(ref))
            want_k.append(ref.decompressed)
        np.testing.assert_array_equal(cache.key_cache[layer].cpu().numpy(), np.concatenate(want_k, 2))
    rep = cache.memory_report()
    assert "Total compressed" in rep and cache.compressed_bytes() > 0 and cache.side_info_bytes() > 0


def test_cache_decode_never_decompresses_gpu(monkeypatch):
    """update() never calls _decompress_chunk (llm/compressed_kv_cache.py:623-660)."""
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache
    calls = []
    orig = CompressedKVCache._decompress_chunk
    monkeypatch.setattr(CompressedKVCache, "_decompress_chunk", lambda self, c: calls.append(1) or orig(self, c))
    cache = CompressedKVCache(bits_per_dim=3)
    for T in (16, 1, 1, 1):
        cache.update(torch.randn(1, 4, T, 64).half().cuda(), torch.randn(1, 4, T, 64).half().cuda(), 0)
    assert calls == []


def test_cache_uncompressible_and_eval_only_gpu():
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache
    cache = CompressedKVCache(bits_per_dim=4)
    a, b = torch.randn(1, 2, 5, 12).half().cuda(), torch.randn(1, 2, 3, 12).half().cuda()
    cache.update(a, a, 0)
    k, v = cache.update(b, b, 0)
    assert torch.equal(k, torch.cat([a, b], 2)) and cache.get_seq_length(0) == 8
    ev = CompressedKVCache(bits_per_dim=5, eval_only_no_entropy=True)
    t = torch.randn(1, 8, 20, 128).half()
    k, _ = ev.update(t.cuda(), t.cuda(), 0)
    from latticequant_amd import codec
    q, s32, s16 = codec.quantize_points(t.cuda(), 5)
    qo = O.quantize_heads(t.float().numpy(), s32.cpu().numpy())
    want = (qo.reshape(8, -1, 8) * s32.cpu().numpy()[:, None, None]).astype(np.float32)
    np.testing.assert_array_equal(k.cpu().numpy(), want.reshape(t.shape).astype(np.float16))
    assert ev.get_seq_length(0) == 20 and ev.compressed_bytes() == 2 * (4 + 1 + 2 * 8)


def test_fixed_rate_merge_gpu():
    """compress_fixed_rate -> fused_decompress_chunk == triton_decompress_chunk ==
    q * scale16 for every vector (packed or fp16 fallback), b = 3, 4, 5."""
    from latticequant_amd.llm.compressed_kv_cache import compress_fixed_rate
    from latticequant_amd.llm.fused_triton_merge import fused_decompress_chunk
    from latticequant_amd.llm.triton_kv_integration import triton_decompress_chunk
    gen = torch.Generator().manual_seed(21)
    t = torch.randn(2, 4, 96, 128, generator=gen)
    t[..., :3] *= 12.0
    t = t.half()
    from latticequant_amd import codec
    q, sc32, sc16 = codec.quantize_points(t.cuda(), 4)
    qo = O.quantize_heads(t.float().numpy(), sc32.cpu().numpy())
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    for b in (3, 4, 5):
        ch = compress_fixed_rate(t.cuda(), bits_per_dim=4, storage_bits=b)
        fused = fused_decompress_chunk(ch).cpu().numpy()
        np.testing.assert_array_equal(fused, triton_decompress_chunk(ch).cpu().numpy())
        s16 = ch.scales.cpu().numpy()          # the fp16-stored scales, widened
        want = (qo.reshape(8, -1, 8) * s16[:, None, None]).astype(np.float32).astype(np.float16).reshape(t.shape)
        np.testing.assert_array_equal(fused, want)
        np.testing.assert_array_equal(ch.repr_mask.cpu().numpy(), O.check_representable(qo, b))
        assert 0 < int(ch.repr_mask.sum()) < ch.n_vectors


def test_compact_index_clamping_gpu(monkeypatch):
    """No host sync by default: out-of-range head indices and masks that select
    more rows than packed / fallback hold are clamped in the kernels (garbage,
    never a fault); LQ_DEBUG_CHECKS=1 restores the host-side ValueErrors."""
    from latticequant_amd.core import triton_dequant as td
    from latticequant_amd.llm.compressed_kv_cache import compress_fixed_rate
    from latticequant_amd.llm.fused_triton_merge import fused_decompress_chunk
    gen = torch.Generator().manual_seed(23)
    packed = torch.randint(0, 256, (64, 4), generator=gen, dtype=torch.uint8).cuda()
    sc = torch.rand(3, generator=gen).cuda()
    hi = torch.zeros(64, dtype=torch.int32)
    hi[:5] = torch.tensor([0, 1, 2, 7, -3], dtype=torch.int32)
    out = td.triton_unpack_e8_4bit(packed, sc, hi.cuda())
    assert torch.equal(out, td.triton_unpack_e8_4bit(packed, sc, hi.clamp(0, 2).cuda()))
    t = torch.randn(1, 2, 64, 128, generator=gen)
    t[..., :3] *= 12.0
    ch = compress_fixed_rate(t.half().cuda(), bits_per_dim=4, storage_bits=4)
    good = fused_decompress_chunk(ch)
    n_pk = int(ch.packed.shape[0])
    assert 1 < n_pk < ch.n_vectors
    ch.packed = ch.packed[:n_pk // 2].clone()          # the mask now selects rows past the end
    bad = fused_decompress_chunk(ch)
    assert bad.shape == good.shape
    monkeypatch.setenv("LQ_DEBUG_CHECKS", "1")
    with pytest.raises(ValueError, match="head_indices"):
        td.triton_unpack_e8_4bit(packed, sc, hi.cuda())
    with pytest.raises(ValueError, match="mask selects"):
        fused_decompress_chunk(ch)


@pytest.mark.parametrize("bits,storage", [(4, 4), (4, 3), (4, 5), (3, 3)])
def test_compact_encode_merge_device_gpu(bits, storage):
    """Sync-free fixed-rate round trip (codec.compact_encode -> compact_merge)
    over 73 tiles of 1024 vectors (the last one partial): packed words, mask,
    fp16 fallback rows, head ids, tile offsets and totals against the oracle
    (quantize_heads / check_representable / pack_e8 at the device's scales),
    and the merged output equal to q * float(scale16)."""
    from latticequant_amd import codec
    gen = torch.Generator().manual_seed(40 + 3 * bits + storage)
    t = torch.randn(1, 3, 24870, 8, generator=gen)          # 74610 vectors: 72 full tiles + a partial one
    t[..., :2] *= 9.0
    t = t.half()
    cb = codec.compact_encode(t.cuda(), bits, storage)
    n_repr, n_oor = codec.compact_counts(cb.totals)
    V = t.numel() // 8
    s32 = cb.scale32.cpu().numpy()
    qo = O.quantize_heads(t.float().numpy(), s32)
    m = O.check_representable(qo, storage)
    assert n_repr == int(m.sum()) and n_oor == V - n_repr and 0 < n_repr < V
    np.testing.assert_array_equal(cb.mask.cpu().numpy().astype(bool), m)
    np.testing.assert_array_equal(cb.packed[:n_repr].cpu().numpy(), O.pack_e8(qo[m], storage))
    bph = V // 3
    heads = np.arange(V) // bph
    np.testing.assert_array_equal(cb.repr_heads[:n_repr].cpu().numpy(), heads[m])
    s16 = cb.scale16.float().cpu().numpy()
    full = (qo * s16[heads][:, None]).astype(np.float32).astype(np.float16)
    np.testing.assert_array_equal(cb.fallback[:n_oor].cpu().numpy(), full[~m])
    tiles = (V + 1023) // 1024
    want_off = np.concatenate([[0], np.cumsum(m.reshape(-1)[:tiles * 1024 - 1024].reshape(tiles - 1, 1024).sum(1))])
    np.testing.assert_array_equal(cb.tile_off.cpu().numpy(), want_off)
    out = codec.compact_merge(cb)
    np.testing.assert_array_equal(out.cpu().numpy().reshape(-1, 8), full)


def _compact_two_ways(x, bits, storage):
    """(scaled, separate): the outputs of lq_compact_encode_scaled and of
    lq_head_scales + lq_compact_encode on one (n_heads, bph, 8) input."""
    from latticequant_amd import _lib as L
    from latticequant_amd import codec
    lib = L.lib()
    nh, bph = x.shape[0], x.shape[1]
    V = nh * bph
    dev = x.device
    dt = L.dtype_code(x.dtype)
    s = L.stream_ptr(dev)
    tiles = (V + 1023) // 1024

    def outs():
        return dict(mask=torch.full((V,), 7, dtype=torch.uint8, device=dev),
                    packed=torch.zeros(V * storage, dtype=torch.uint8, device=dev),
                    fallback=torch.zeros(V * 8, dtype=torch.float16, device=dev),
                    heads=torch.full((V,), -1, dtype=torch.int32, device=dev),
                    tile_off=torch.full((tiles,), -1, dtype=torch.int64, device=dev),
                    totals=torch.full((3,), -1, dtype=torch.int64, device=dev))

    a = outs()
    a["sigma2"] = torch.full((nh,), -1.0, device=dev)
    a["scale32"] = torch.full((nh,), -1.0, device=dev)
    a["scale16"] = torch.zeros(nh, dtype=torch.float16, device=dev)
    a["scale16f"] = torch.full((nh,), -1.0, device=dev)
    work = torch.full((lib.lq_compact_encode_scaled_workspace(nh, bph),), 0xAB, dtype=torch.uint8, device=dev)
    L.check(lib.lq_compact_encode_scaled(x.data_ptr(), dt, nh, bph, bits, storage, a["sigma2"].data_ptr(),
                                         a["scale32"].data_ptr(), a["scale16"].data_ptr(), a["scale16f"].data_ptr(),
                                         a["mask"].data_ptr(), a["packed"].data_ptr(), a["fallback"].data_ptr(),
                                         a["heads"].data_ptr(), a["tile_off"].data_ptr(), a["totals"].data_ptr(),
                                         work.data_ptr(), s), "lq_compact_encode_scaled")
    b = outs()
    bits_t = torch.full((1,), bits, dtype=torch.int32, device=dev)
    hw = torch.empty(4096 + nh, dtype=torch.float64, device=dev)
    b["sigma2"] = torch.empty(nh, device=dev)
    b["scale32"] = torch.empty(nh, device=dev)
    b["scale16"] = torch.empty(nh, dtype=torch.float16, device=dev)
    fd = torch.empty(nh, dtype=torch.int32, device=dev)
    L.check(lib.lq_head_scales(x.data_ptr(), dt, 1, nh, bph, bits_t.data_ptr(), hw.data_ptr(), b["sigma2"].data_ptr(),
                               b["scale32"].data_ptr(), b["scale16"].data_ptr(), fd.data_ptr(), s), "lq_head_scales")
    wb = torch.full((lib.lq_compact_encode_workspace(V),), 0xAB, dtype=torch.uint8, device=dev)
    L.check(lib.lq_compact_encode(x.data_ptr(), dt, nh, bph, b["scale32"].data_ptr(), fd.data_ptr(),
                                  b["scale16"].data_ptr(), storage, b["mask"].data_ptr(), b["packed"].data_ptr(),
                                  b["fallback"].data_ptr(), b["heads"].data_ptr(), b["tile_off"].data_ptr(),
                                  b["totals"].data_ptr(), wb.data_ptr(), s), "lq_compact_encode")
    b["scale16f"] = b["scale16"].float()
    for d in (a, b):
        n_repr, n_oor = codec.compact_counts(d["totals"])
        d["packed"] = d["packed"][:n_repr * storage]
        d["heads"] = d["heads"][:n_repr]
        d["fallback"] = d["fallback"][:n_oor * 8]
    return a, b


@pytest.mark.parametrize("nh,bph,dtype,bits,storage", [
    (8, 32768, torch.float16, 4, 4),      # C1's shape: one head per tile
    (3, 1025, torch.float16, 4, 3),       # every tile but one spans two heads
    (5, 1024, torch.bfloat16, 3, 3),      # bph at the limit
    (1, 65536, torch.float32, 5, 5),      # one head: 128 sigma^2 parts (two waves of lanes)
    (4, 3000, torch.float16, 4, 5),       # a zero head (scale 1) among others
])
def test_compact_encode_scaled_equals_separate_gpu(nh, bph, dtype, bits, storage):
    """lq_compact_encode_scaled (scales finalised inside the encoder) writes
    the same sigma^2, scales, fp16 scales, mask, packed words, fallback rows,
    head ids, tile offsets and totals as lq_head_scales + lq_compact_encode,
    byte for byte, with float(scale16) beside them; twice in a row on one
    workspace (its look-back words are cleared by the call)."""
    gen = torch.Generator().manual_seed(nh * 7 + bph)
    x = torch.randn(nh, bph, 8, generator=gen)
    x[:, :, :2] *= 6.0
    if nh == 4:
        x[2] = 0.0
    x = x.to(dtype).cuda()
    for _ in range(2):
        a, b = _compact_two_ways(x, bits, storage)
        for k in a:
            assert torch.equal(a[k].cpu(), b[k].cpu()), k
    n_repr = int(a["totals"][0])
    assert 0 < n_repr < nh * bph


def test_compact_encode_scaled_rejects_short_heads_gpu():
    """Fewer than 1024 vectors per head: LQ_ERR_ARG (a tile could span more
    than two heads); codec.compact_encode then takes the separate path and
    still matches the oracle."""
    from latticequant_amd import _lib as L
    from latticequant_amd import codec
    lib = L.lib()
    x = torch.randn(4, 1023, 8).half().cuda()
    z = torch.zeros(16, dtype=torch.int64, device="cuda")
    rc = lib.lq_compact_encode_scaled(x.data_ptr(), L.LQ_F16, 4, 1023, 4, 4, None, z.data_ptr(), z.data_ptr(),
                                      z.data_ptr(), z.data_ptr(), z.data_ptr(), z.data_ptr(), None, z.data_ptr(),
                                      z.data_ptr(), z.data_ptr(), L.stream_ptr())
    assert rc == -1   # LQ_ERR_ARG
    cb = codec.compact_encode(x.view(1, 4, 1023, 8), 4)
    qo = O.quantize_heads(x.view(1, 4, 1023, 8).float().cpu().numpy(), cb.scale32.cpu().numpy())
    np.testing.assert_array_equal(cb.mask.cpu().numpy().astype(bool), O.check_representable(qo, 4))
