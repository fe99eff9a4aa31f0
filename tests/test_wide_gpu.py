"""Wide-symbol path (alphabets up to L = 1024 symbols): heavy-tailed keys as in
the layer-wise allocation workload (K Student-t nu = 3 with 8 outlier channels
x20, V N(0, 1), rates 3 / 4 / 5 bits per dimension).

Parity bar: the decoded chunk equals the oracle's decompress_chunk bit for bit
(lossless coding of the same lattice points), and the table, bitstream words,
state and bit count of every stream equal the oracle's (numpy's argsort tie
order included, above 256 symbols too).  Where an alphabet exceeds 1024
symbols (the reference's table normalisation never terminates there,
core/gpu_ans.py:73-84) the chunk is escaped -- coarse symbols s >> k through
the same tables and streams, k raw low bits per vector -- a format of this
build, compared with the oracle's restatement of it (parity unpinned by the
reference); with escape=False it raises AlphabetError."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def student_k(seed, B=1, H=4, T=1024, hd=128, n_out=8, mult=20.0):
    rng = np.random.default_rng(seed)
    k = rng.standard_t(3.0, size=(B, H, T, hd)).astype(np.float32)
    for h in range(H):
        ch = rng.permutation(hd)[:n_out]
        k[:, h, :, ch] *= mult
    return k.astype(np.float16)


def oracle_alphabets(t16, bits, s32):
    """Alphabet sizes range(min-2, max+2) of every present stream, as _compress_tensor forms them."""
    q = O.quantize_heads(t16.astype(np.float32), s32)
    coset, free, c8h = O.e8_to_symbols(q)
    syms = np.concatenate([free, c8h[:, None]], 1)
    sizes = []
    for c in (0, 1):
        sc = syms[coset == c]
        for i in range(8 if len(sc) else 0):
            sizes.append(int(sc[:, i].max() - sc[:, i].min() + 5))
    return sizes


def check_chunk(enc, c, ch):
    """Every stream of chunk c equals the oracle's; returns the widest alphabet."""
    from latticequant_amd import codec
    streams = codec.chunk_streams_host(enc, c)
    assert len(streams) == len(ch.streams)
    widest = 0
    for sd, so in zip(streams, ch.streams):
        assert (sd["coset"], sd["idx"], sd["n"]) == (so.coset, so.idx, so.n_symbols)
        assert sd["lo"] == so.table.alphabet[0] and len(sd["freqs"]) == len(so.table.freqs)
        assert int(sd["freqs"].sum()) == O.L and (sd["freqs"] >= 1).all()
        assert sd["status"] == 0
        np.testing.assert_array_equal(sd["freqs"], so.table.freqs)
        np.testing.assert_array_equal(sd["words"], so.words)
        assert sd["state"] == so.state and sd["n_bits"] == so.n_bits
        widest = max(widest, len(sd["freqs"]))
    return widest


def check_escape(enc, c, ch):
    """Chunk c's escape shifts and low-bit words equal the oracle's."""
    esc = enc.escape
    if ch.esc_k is None:
        assert esc is None or not esc.k_host[c].any()
        return
    assert esc is not None
    np.testing.assert_array_equal(esc.k_host[c], ch.esc_k)
    fine = esc.fine.cpu().numpy().view(np.uint32)
    off = esc.off.cpu().numpy()
    for j, words in ch.fine.items():
        o = int(off[8 * c + j])
        np.testing.assert_array_equal(fine[o:o + words.size], words, err_msg=f"coordinate {j}")


@pytest.mark.parametrize("bits,seed", [(3, 0), (3, 1), (4, 0), (4, 1), (5, 2)])
def test_wide_chunk_vs_oracle_gpu(bits, seed):
    from latticequant_amd import codec
    t = student_k(seed)
    s32, _ = O.cache_scales(O.head_sigma2(t.astype(np.float32)), bits)
    sizes = oracle_alphabets(t, bits, s32)
    x = torch.from_numpy(t).cuda()[None]
    assert max(sizes) > 264, "case should need the wide path"
    if max(sizes) > O.L:
        with pytest.raises(codec.AlphabetError):
            codec.encode_batch(x, bits, scale32=torch.from_numpy(s32), escape=False)
    enc, deq = codec.encode_batch(x, bits, scale32=torch.from_numpy(s32), deq_out=True)
    assert enc.extra["wide"]
    ch = O.compress_chunk(t, bits, scales_f32=s32, escape=True)
    assert (ch.esc_k is not None) == (max(sizes) > O.L)
    check_chunk(enc, 0, ch)
    check_escape(enc, 0, ch)
    np.testing.assert_array_equal(deq[0].cpu().numpy(), ch.decompressed)
    np.testing.assert_array_equal(codec.decode_batch(enc)[0].cpu().numpy(), O.decompress_chunk(ch))


def test_wide_forced_equals_int8_gpu():
    """On int8-range data the wide path writes the same chunk as the int8 path."""
    from latticequant_amd import codec
    g = torch.Generator().manual_seed(4)
    x = torch.randn(3, 1, 4, 64, 128, generator=g).half().cuda()
    a, _ = codec.encode_batch(x, [3, 4, 5], wide=False)
    b, _ = codec.encode_batch(x, [3, 4, 5], wide=True)
    assert not a.extra["wide"] and b.extra["wide"]
    assert torch.equal(a.words[:-2], b.words[:-2])   # the last two words are the decoder's read-ahead slack
    for f in ("coset_bits", "blk_n1", "blk_off", "blk_state", "stream_nbits", "stream_state", "chunk_words"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f
    ta, tb = codec.host_tables(a), codec.host_tables(b)
    for (la, na, sa, _, fa), (lb, nb, sb, _, fb) in zip(ta, tb):
        assert (la, na, sa) == (lb, nb, sb) and np.array_equal(fa, fb)
    assert torch.equal(codec.decode_batch(a), codec.decode_batch(b))


def test_int8_overflow_flag_without_auto_gpu():
    """wide=False leaves an int8 overflow in the status instead of re-encoding."""
    from latticequant_amd import _lib as L
    from latticequant_amd import codec
    x = torch.from_numpy(student_k(0)).cuda()[None]
    enc, _ = codec.encode_batch(x, 3, wide=False, exact_size=False)
    assert int(enc.status[0]) & L.LQ_ST_SYM_OVERFLOW


def test_variable_rate_cache_heavy_tailed_gpu():
    """Layer-wise rates on heavy-tailed K: each chunk equals the oracle's at its
    rate (wide path where needed, escaped where an alphabet exceeds L, which
    the reference never completes).  update() writes without host syncs; the
    first read of a chunk settles it."""
    from latticequant_amd.allocation.eval_alloc import VariableRateKVCache, cyclic_schedule
    sched = cyclic_schedule(3, seed=0)   # 3, 4, 5 bits
    cache = VariableRateKVCache(sched, eval_only_no_entropy=False)
    rng = np.random.default_rng(11)
    escaped = 0
    for layer in range(3):
        k = student_k(100 + layer)
        v = rng.standard_normal((1, 4, 1024, 128)).astype(np.float16)
        b = sched[layer]["K"]
        kk = torch.from_numpy(k).cuda()
        cache.update(kk, torch.from_numpy(v).cuda(), layer)
        ck = cache._comp_keys[layer].chunks[-1]
        s32 = ck.encoded.scale32.cpu().numpy()
        ch = O.compress_chunk(k, b, scales_f32=s32, escape=True)
        escaped += ch.esc_k is not None
        check_chunk(ck.encoded, 0, ch)
        check_escape(ck.encoded, 0, ch)
        np.testing.assert_array_equal(cache._decompress_chunk(ck).cpu().numpy(), O.decompress_chunk(ch))
        cv = cache._comp_values[layer].chunks[-1]
        chv = O.compress_chunk(v, sched[layer]["V"], scales_f32=cv.encoded.scale32.cpu().numpy())
        np.testing.assert_array_equal(cv.gpu_bitstream.cpu().numpy().view(np.uint32), chv.bitstream)
    assert escaped >= 1 and len(cache._comp_keys[0].chunks) == 1


def test_pending_escape_plan_decodes_like_resolved_gpu(monkeypatch):
    """The wide path's escape plan reaches the host only when first read, and
    decode_batch does not wait for it: an unread plan takes the escaped
    decoder, which reads the shifts on the device (a chunk with every k_j = 0
    decodes plainly).  Both forms give the same rows, for a batch with an
    escaped chunk and one without; reading the plan trims the fine words to
    the batch's own."""
    from latticequant_amd import codec
    print("pending escape plan", flush=True)
    # 4 bits: seed 0's widest alphabet is 538 symbols, seed 1's 1130 (escaped);
    # 3 bits, seed 2: 360 (wide, nothing escaped)
    x_esc = torch.from_numpy(np.stack([student_k(0), student_k(1)])).cuda()
    x_plain = torch.from_numpy(student_k(2)[None]).cuda()
    for x, bits in ((x_esc, 4), (x_plain, 3)):
        enc, _ = codec.encode_batch(x, bits, exact_size=False, wide=True)
        monkeypatch.setattr(codec.Escape, "ready", lambda self: False)
        pend = codec.decode_batch(enc)
        monkeypatch.undo()
        bound = enc.extra["esc"].fine.numel()
        esc = enc.escape   # reads the plan back
        res = codec.decode_batch(enc)
        torch.cuda.synchronize()
        assert torch.equal(pend, res)
        if esc is None:
            assert bits == 3
        else:
            used = int((16 * enc.nblk * esc.k_host.astype(np.int64)).sum())
            assert esc.any() and esc.fine.numel() == used + 1 < bound
