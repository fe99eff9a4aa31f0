"""GPU parity of the E8 + rANS chunk codec against the CPU oracle.

Bit-exact: lattice points, symbols, coset bitmap, tables, bitstream words,
final states, n_bits; fp16 outputs bit-exact (the contract allows 1 ulp)."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
pytestmark = pytest.mark.gpu


def _lq():
    from latticequant_amd import codec, _lib
    return codec, _lib


def _e8_gpu(x, mode):
    codec, L = _lq()
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    out = torch.empty_like(xt)
    L.check(L.lib().lq_e8_encode_f32(xt.data_ptr(), xt.shape[0], mode, out.data_ptr(), L.stream_ptr()), "e8")
    return out.cpu().numpy()


def test_e8_golden_gpu():
    g = np.load(os.path.join(G, "e8.npz"))
    np.testing.assert_array_equal(_e8_gpu(g["x"], 0), g["e8"])
    np.testing.assert_array_equal(_e8_gpu(g["x"], 1), g["d8"])


def test_e8_random_vs_oracle_gpu():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((1 << 18, 8)) * rng.choice([0.3, 3, 30], size=(1 << 18, 1))).astype(np.float32)
    np.testing.assert_array_equal(_e8_gpu(x, 0), O.encode_e8(x))


def _compare_chunk(enc, c, ch, check_tables=True):
    codec, L = _lq()
    streams = codec.chunk_streams_host(enc, c)
    assert len(streams) == len(ch.streams)
    for sg, so in zip(streams, ch.streams):
        assert (sg["coset"], sg["idx"], sg["n"]) == (so.coset, so.idx, so.n_symbols)
        assert sg["lo"] == so.table.alphabet[0]
        if check_tables:
            np.testing.assert_array_equal(sg["freqs"], so.table.freqs)
        assert sg["n_bits"] == so.n_bits and sg["state"] == so.state
        np.testing.assert_array_equal(sg["words"], so.words)
    nb = (ch.n_vectors + 7) // 8
    np.testing.assert_array_equal(enc.coset_bits[c].cpu().numpy()[:nb], ch.coset_packed)
    base = int(enc.chunk_base[c]); nw = int(enc.chunk_words[c])
    np.testing.assert_array_equal(enc.words[base:base + nw].cpu().numpy().view(np.uint32), ch.bitstream)


def test_chunk_golden_cases_gpu():
    """The reference's own _compress_tensor outputs (tests/golden/cache.npz)."""
    codec, L = _lq()
    g = np.load(os.path.join(G, "cache.npz"))
    for ci in range(int(g["n_cases"])):
        p = f"c{ci}_"
        t = g[p + "input"]
        bits = int(g[p + "bits"])
        ch = O.compress_chunk(t, bits)   # oracle == reference on these cases (tests/test_oracle.py)
        x = torch.from_numpy(t).cuda()[None]
        enc, deq = codec.encode_batch(x, bits, scale32=torch.from_numpy(ch.scales_f32), deq_out=True)
        assert int(enc.status.item()) == 0
        np.testing.assert_array_equal(deq[0].cpu().numpy(), g[p + "decompressed"])
        _compare_chunk(enc, 0, ch)
        np.testing.assert_array_equal(codec.decode_batch(enc)[0].cpu().numpy(), g[p + "rebuilt"])
        # scales computed on the device
        enc2, _ = codec.encode_batch(x, bits)
        np.testing.assert_array_equal(enc2.scale16.cpu().numpy(), g[p + "scales"])


@pytest.mark.parametrize("shape,bits,seed", [((1, 8, 256, 128), 4, 1), ((1, 8, 1024, 128), 3, 2),
                                             ((2, 4, 300, 64), 5, 3), ((1, 8, 8192, 128), 4, 4)])
def test_chunk_random_vs_oracle_gpu(shape, bits, seed):
    codec, L = _lq()
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(*shape, generator=g)
    ch_idx = torch.randperm(shape[-1], generator=g)[:4]
    t[..., ch_idx] *= 10.0
    t = t.to(torch.float16)
    tn = t.numpy()
    ch = O.compress_chunk(tn, bits)
    enc, deq = codec.encode_batch(t.cuda()[None], bits, scale32=torch.from_numpy(ch.scales_f32), deq_out=True)
    assert int(enc.status.item()) == 0
    np.testing.assert_array_equal(deq[0].cpu().numpy(), ch.decompressed)
    _compare_chunk(enc, 0, ch)
    np.testing.assert_array_equal(codec.decode_batch(enc)[0].cpu().numpy(), O.decompress_chunk(ch))
    # device sigma^2 agrees with the oracle's float64 mean to fp32 rounding
    enc2, _ = codec.encode_batch(t.cuda()[None], bits)
    np.testing.assert_allclose(enc2.sigma2.cpu().numpy(), O.head_sigma2(tn), rtol=2e-7)


def test_chunk_batch_and_roundtrip_gpu():
    """Several chunks per call, mixed bit rates, bf16 input; decode(encode) == q * scale16."""
    codec, L = _lq()
    g = torch.Generator().manual_seed(11)
    x = torch.randn(6, 1, 4, 96, 128, generator=g).to(torch.bfloat16)
    bits = [3, 4, 5, 4, 3, 5]
    enc, deq = codec.encode_batch(x.cuda(), bits, deq_out=True)
    assert enc.status.cpu().numpy().tolist() == [0] * 6
    out = codec.decode_batch(enc, out_dtype=torch.bfloat16)
    for c in range(6):
        sc32 = enc.scale32.view(6, -1)[c].cpu().numpy()
        ch = O.compress_chunk(x[c].float().numpy(), bits[c], scales_f32=sc32)
        _compare_chunk(enc, c, ch)
        # bf16 read path: float(q) * float(scale16) rounded to bf16
        q = torch.from_numpy(O.quantize_heads(x[c].float().numpy(), sc32))
        sc = enc.scale16.view(6, -1)[c].float().cpu()
        want = (q.view(4, -1, 8) * sc[:, None, None]).to(torch.bfloat16).view(1, 4, 96, 128)
        assert torch.equal(out[c].cpu(), want)


def test_prefilled_arena_gpu():
    """Bound-sized arena full of ones (exact_size=False, words_out): every word
    of every chunk, the streams' trailing zero words included, is written by
    the encoder; chunk bases are the exclusive prefix of the word counts."""
    codec, L = _lq()
    g = torch.Generator().manual_seed(23)
    x = torch.randn(3, 1, 4, 200, 128, generator=g).half()
    V = 4 * 200 * 128 // 8
    arena = torch.full((codec.words_bound(3, V),), -1, dtype=torch.int32, device="cuda")
    enc, _ = codec.encode_batch(x.cuda(), 4, exact_size=False, words_out=arena, wide=False)
    cw = enc.chunk_words.cpu().numpy()
    np.testing.assert_array_equal(enc.chunk_base.cpu().numpy(), np.cumsum(cw) - cw)
    for c in range(3):
        sc32 = enc.scale32.view(3, -1)[c].cpu().numpy()
        _compare_chunk(enc, c, O.compress_chunk(x[c].float().numpy(), 4, scales_f32=sc32))


def test_empty_coset_and_zero_head_gpu():
    codec, L = _lq()
    t = torch.zeros(1, 2, 8, 64, dtype=torch.float16)
    t[0, 1] = torch.randn(8, 64).half()
    ch = O.compress_chunk(t.numpy(), 4)
    enc, deq = codec.encode_batch(t.cuda()[None], 4, deq_out=True)
    np.testing.assert_array_equal(enc.scale16.cpu().numpy(), ch.scales)
    _compare_chunk(enc, 0, ch)
    np.testing.assert_array_equal(codec.decode_batch(enc)[0].cpu().numpy(), O.decompress_chunk(ch))


@pytest.mark.parametrize("frac1,seed", [(0.02, 21), (0.002, 22)])
def test_sparse_coset_streams_gpu(frac1, seed):
    """Lattice-exact input (scale 1): D8 points, plus a small fraction of
    D8 + 1/2 points, so the coset-1 streams have blocks of a few symbols or
    none: stream words then span several blocks (bitstream assembly's
    continuation across short and empty blocks) and the decoder walks long
    runs of empty bitmap words.  Bit-exact against the oracle."""
    codec, L = _lq()
    rng = np.random.default_rng(seed)
    shape = (1, 8, 1024, 128)
    y = rng.integers(-3, 4, size=shape[:-1] + (16, 8))
    y[..., 7] += y.sum(-1) & 1                       # even coordinate sum: D8
    half = rng.random(shape[:-1] + (16,)) < frac1    # these vectors move to D8 + 1/2
    x = y.astype(np.float32) + 0.5 * half[..., None]
    t = torch.from_numpy(x.reshape(shape).astype(np.float16))
    sc = np.ones(8, np.float32)
    ch = O.compress_chunk(t.numpy(), 4, scales_f32=sc)
    enc, _ = codec.encode_batch(t.cuda()[None], 4, scale32=torch.from_numpy(sc))
    assert int(enc.status.item()) == 0
    n1 = int(enc.blk_n1.sum().item())
    assert n1 == int(half.sum())
    if frac1 < 0.01:
        assert int((enc.blk_n1 == 0).sum().item()) > 0   # some blocks hold no coset-1 symbol
    _compare_chunk(enc, 0, ch)
    np.testing.assert_array_equal(codec.decode_batch(enc)[0].cpu().numpy(), O.decompress_chunk(ch))


def test_fp32_ragged_chunk_vs_oracle_gpu():
    """fp32 input (IEEE division in the quantizer, no fast path), a vector count
    that is not a multiple of the 512-vector block, heavy-tailed values: the
    bitstream is bit-exact and the fp32 read path is q * float(scale16)."""
    codec, L = _lq()
    g = torch.Generator().manual_seed(31)
    x = (torch.randn(1, 2, 4, 77, 128, generator=g) * torch.rand(1, 2, 4, 77, 1, generator=g) * 3).float()
    x[..., :2] *= 25.0
    enc, _ = codec.encode_batch(x.cuda(), 4)
    assert int(enc.status.item()) == 0
    sc32 = enc.scale32.cpu().numpy()
    ch = O.compress_chunk(x[0].numpy(), 4, scales_f32=sc32)
    _compare_chunk(enc, 0, ch)
    out = codec.decode_batch(enc, out_dtype=torch.float32)
    np.testing.assert_array_equal(out[0].cpu().numpy(), O.decompress_chunk(ch, out_dtype=np.float32))
    np.testing.assert_allclose(enc.sigma2.cpu().numpy(), O.head_sigma2(x[0].numpy()), rtol=2e-7)


def test_long_stream_tiled_scan_vs_oracle_gpu():
    """A chunk with more than 4096 blocks per stream (2 x 73728 tokens x 128:
    4608 blocks, one full 4096-block scan tile and a partial one): the
    block offsets come from the tiled scan; bitstream, offsets and decode are
    bit-exact against the oracle."""
    codec, L = _lq()
    x = torch.randn(1, 1, 2, 73728, 128, generator=torch.Generator().manual_seed(73)).half()
    enc, _ = codec.encode_batch(x.cuda(), 4)
    assert enc.nblk > 4096 and int(enc.status.item()) == 0
    ch = O.compress_chunk(x[0].numpy(), 4, scales_f32=enc.scale32.cpu().numpy())
    _compare_chunk(enc, 0, ch)
    # per stream the block offsets rise by each block's bit count and end at n_bits
    off = enc.blk_off.view(16, -1).cpu().numpy().astype(np.int64)
    nb = enc.stream_nbits.cpu().numpy()
    assert (np.diff(off, axis=1) >= 0).all() and (off[:, 0] == 0).all() and (off[:, -1] <= nb).all()
    np.testing.assert_array_equal(codec.decode_batch(enc)[0].cpu().numpy(), O.decompress_chunk(ch))


def test_quantize_deq_matches_quantize_batch_gpu():
    """lq_quantize_deq (the scales and the dequantised rows of a small update
    in one call, by-products in the caller's scratch) returns what
    quantize_batch returns, over calls in a row that share one scratch (the
    later ones smaller, so stale scratch is read back only if the kernel
    wrongly depends on it), fp16 / bf16 / fp32, per-chunk rates, and the
    dequantised rows equal the oracle's."""
    codec, _ = _lq()
    sc = codec.QuantizeScratch()
    cases = [((2, 1, 8, 40, 128), torch.float16, 4), ((2, 1, 8, 1, 128), torch.float16, [3, 5]),
             ((2, 2, 4, 3, 64), torch.bfloat16, 4), ((1, 1, 2, 1, 128), torch.float32, 5)]
    for shape, dt, bits in cases:
        print(f"case {shape} {dt} {bits}", flush=True)
        x = torch.randn(*shape, generator=torch.Generator().manual_seed(sum(shape))).mul(3.0).to(dt).cuda()
        got = codec.quantize_deq(x, bits, sc)
        want = codec.quantize_batch(x, bits, with_sigma2=True)
        for g, w, name in zip(got, want, ("scale32", "scale16", "deq", "sigma2")):
            assert torch.equal(g, w), name
    # the oracle's dequantised rows for the last fp16 case
    x = torch.randn(2, 1, 8, 1, 128, generator=torch.Generator().manual_seed(3)).half()
    s32, _, deq, _ = codec.quantize_deq(x.cuda(), 4, sc)
    for c in range(2):
        ch = O.compress_chunk(x[c].numpy(), 4, scales_f32=s32.view(2, -1)[c].cpu().numpy())
        np.testing.assert_array_equal(deq[c].cpu().numpy(), ch.decompressed)


@pytest.mark.parametrize("peak", [125.6, 126.4, 127.3, 128.6])
def test_int8_range_check_near_its_bound_gpu(peak):
    """The quantizer checks the int8 range of a vector's symbols only when the
    vector's max |x / scale| reaches 126 (below that every coordinate, flip
    included, lies within +-127).  Vectors with one coordinate at +-peak times
    its head's scale (the scale settled by iterating, since the peaks move
    sigma^2), the rest Gaussian: at 125.6 the check is skipped with symbols
    up to +-126, at 126.4 and 127.3 it runs with symbols up to -128 / 127 (in
    range), at 128.6 a symbol reaches 129.  The overflow flag is set exactly
    when the oracle's symbols leave int8, and the chunk equals the oracle's
    when they do not."""
    codec, L = _lq()
    rng = np.random.default_rng(int(peak * 10))
    x = rng.standard_normal((1, 2, 256, 128)).astype(np.float32)
    sel = [(0, 5, 3), (0, 17, 64 + 7), (1, 40, 8 * 5 + 1), (1, 63, 127), (0, 130, 12), (1, 200, 100)]
    for _ in range(12):
        s = O.compress_chunk(x.astype(np.float16).astype(np.float32), 4).scales_f32
        for k, (h, t, d) in enumerate(sel):
            x[0, h, t, d] = (peak if k % 2 == 0 else -peak) * s[h]
    xh = x.astype(np.float16)
    enc, _ = codec.encode_batch(torch.from_numpy(xh).cuda()[None], 4, wide=False, exact_size=False)
    # the oracle at the device's scales (sigma^2 sums in another order can move
    # a scale's last bit, and with it a point near a decision boundary)
    sc32 = enc.scale32.cpu().numpy()
    ch = O.compress_chunk(xh.astype(np.float32), 4, scales_f32=sc32)
    ts = [abs(float(xh[0, h, t, d]) / float(sc32[h])) for h, t, d in sel]
    assert max(abs(t - peak) for t in ts) < 0.1
    lo = min(st.table.alphabet[0] + 2 for st in ch.streams)    # alphabets are padded by 2 on each side
    hi = max(st.table.alphabet[-1] - 2 for st in ch.streams)
    over = lo < -128 or hi > 127
    assert over == (peak > 128)
    assert bool(int(enc.status[0]) & L.LQ_ST_SYM_OVERFLOW) == over
    if not over:
        _compare_chunk(enc, 0, ch)
