"""Wire / on-disk format of a compressed chunk batch (codec.to_bytes / from_bytes).

CPU tests exercise the container on a synthetic batch (field round trip,
table rebuild, corruption and version checks); the GPU tests round-trip real
encoded batches and check that the restored batch decodes bit-exactly."""
import io
import os

import numpy as np
import pytest
import torch

from latticequant_amd import codec
from latticequant_amd import _lib as L


def _fake_batch(C=2, nh=2, bph=1000, seed=0):
    """A structurally valid EncodedBatch on the CPU: random tables, bitmap and
    words, with every cross-field rule of the format kept (the coset-1 counts
    are the bitmap's, a coset's streams are present exactly when it holds
    vectors -- chunk 1 has no coset-1 vector --, the word offsets follow the
    merged layout, checkpoints are non-decreasing from 0 within n_bits).  bph
    is not a multiple of the block size, so the last block is partial."""
    rng = np.random.default_rng(seed)
    S, B = L.LQ_STREAMS, L.LQ_BLK
    nv = nh * bph
    nb = (nv + B - 1) // B
    bits = (rng.random((C, nb, B)) < 0.5).astype(np.uint8)
    bits[:, np.arange(B)[None, :] >= np.minimum(B, nv - np.arange(nb) * B)[:, None]] = 0
    bits[1] = 0
    coset_bits = np.packbits(bits, axis=2, bitorder="little").reshape(C, -1)
    n1 = bits.sum(2).astype(np.int32)
    tot1 = n1.sum(1)
    present = np.zeros((C, S), bool)
    present[:, 8:] = (tot1 > 0)[:, None]
    present[:, :8] = (nv - tot1 > 0)[:, None]
    tab = np.zeros((C * S, L.TABLE_BYTES // 4), np.uint32)
    nbits = np.zeros((C, S), np.int64)
    off = np.zeros((C, S, nb), np.uint32)
    st = np.full((C, S, nb), L.LQ_L, np.int64)
    for c in range(C):
        for k in range(S):
            if not present[c, k]:
                continue
            i = c * S + k
            n = int(rng.integers(3, 40))
            # every symbol at least once, the rest at random: sums to L, every f >= 1
            f = np.bincount(np.concatenate([np.arange(n), rng.integers(0, n, L.LQ_L - n)]), minlength=n)
            cum = np.cumsum(f) - f
            bl = np.array([int(v).bit_length() for v in f], np.uint32)
            tab[i, :4] = np.array([-(n // 2), n, int(rng.integers(1, 999)), 0], np.int32).view(np.uint32)
            tab[i, 4:4 + n] = f.astype(np.uint32) | (cum.astype(np.uint32) << 11) | ((11 - bl) << 21)
            nbits[c, k] = int(rng.integers(0, 5000))
            off[c, k] = np.sort(np.concatenate([[0], rng.integers(0, nbits[c, k] + 1, nb - 1)]))
            st[c, k] = rng.integers(L.LQ_L, 2 * L.LQ_L, nb)
    per = np.where(present, (nbits + 31) // 32 + 1, 0)
    woff = np.cumsum(per, 1) - per
    cw = per.sum(1)
    words = rng.integers(0, 2 ** 32, int(cw.sum()) + 7, dtype=np.uint64).astype(np.uint32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    return codec.EncodedBatch(
        n_chunks=C, n_heads=nh, bph=bph, shape=(1, nh, bph * 8 // 64, 64), bits=T(np.full(C, 4, np.int32)),
        scale32=T(rng.random(C * nh).astype(np.float32)), scale16=T(rng.random(C * nh).astype(np.float16)),
        sigma2=T(rng.random(C * nh).astype(np.float32)),
        coset_bits=T(coset_bits), blk_n1=T(n1),
        tables=T(tab.view(np.uint8).reshape(-1)),
        blk_off=T(off.reshape(-1).view(np.int32)),
        blk_state=T(st.reshape(-1).astype(np.uint16).view(np.int16)),
        stream_nbits=T(nbits.reshape(-1)), stream_state=T(rng.integers(1024, 2048, C * S).astype(np.int32)),
        stream_woff=T(woff.reshape(-1)), chunk_words=T(cw.astype(np.int64)),
        chunk_base=T((np.cumsum(cw) - cw + 3).astype(np.int64)), words=T(words.view(np.int32)),
        status=T(np.zeros(C, np.int32)))


def _meaningful_tables(enc):
    t = enc.tables.view(torch.int32).view(-1, L.TABLE_BYTES // 4).cpu().numpy()
    return [t[i, :4 + t[i, 1]].copy() for i in range(t.shape[0])]


def test_wire_round_trip_fields_cpu():
    e = _fake_batch()
    b = codec.to_bytes(e)
    r = codec.from_bytes(b, device="cpu")
    C, S, nb = e.n_chunks, L.LQ_STREAMS, e.nblk
    for name in ("bits", "status", "scale32", "scale16", "sigma2", "coset_bits", "blk_n1", "stream_nbits",
                 "stream_state", "stream_woff", "chunk_words"):
        assert torch.equal(getattr(r, name).cpu().view(-1), getattr(e, name).view(-1)), name
    for a, b2 in zip(_meaningful_tables(e), _meaningful_tables(r)):
        assert np.array_equal(a, b2)
    ew = e.words.numpy().view(np.uint32)
    rw = r.words.numpy().view(np.uint32)
    for c in range(C):
        b0, n = int(e.chunk_base[c]), int(e.chunk_words[c])
        r0 = int(r.chunk_base[c])
        assert np.array_equal(ew[b0:b0 + n], rw[r0:r0 + n])
    # checkpoints of present streams survive; absent streams read as empty
    nsym = e.tables.view(torch.int32).view(-1, L.TABLE_BYTES // 4)[:, 1].numpy()
    eo = e.blk_off.numpy().reshape(C * S, nb)
    ro = r.blk_off.numpy().reshape(C * S, nb)
    assert np.array_equal(eo[nsym > 0], ro[nsym > 0])
    assert (ro[nsym == 0] == 0).all()


def test_wire_rejects_corruption_and_versions_cpu(tmp_path):
    e = _fake_batch(seed=1)
    b = bytearray(codec.to_bytes(e))
    p = tmp_path / "batch.lq"
    assert codec.save_batch(p, e) == len(b)
    assert codec.load_batch(p, device="cpu").n_chunks == e.n_chunks
    bad = bytearray(b)
    bad[len(bad) // 2] ^= 0x40
    with pytest.raises(codec.WireFormatError, match="checksum"):
        codec.from_bytes(bytes(bad), device="cpu")
    with pytest.raises(codec.WireFormatError):
        codec.from_bytes(bytes(b[:100]), device="cpu")
    with pytest.raises(codec.WireFormatError, match="not an"):
        codec.from_bytes(b"XXXXXXXX" + bytes(b[8:]), device="cpu")
    v2 = bytearray(b)
    v2[8:12] = np.uint32(99).tobytes()
    with pytest.raises(codec.WireFormatError, match="version"):
        codec.from_bytes(bytes(v2), device="cpu")


def _with_escape(e, seed=5):
    """The fake batch with an escape on chunk 0 (coordinates 1 and 7)."""
    rng = np.random.default_rng(seed)
    C, nb = e.n_chunks, e.nblk
    kh = np.zeros((C, 8), np.int32)
    kh[0, 1], kh[0, 7] = 2, 3
    per = 16 * nb * kh.astype(np.int64).reshape(-1)
    off = np.cumsum(per) - per
    fine = rng.integers(0, 2**31, int(per.sum()) + 1).astype(np.int32)
    e.extra["esc"] = codec.Escape(k=torch.from_numpy(kh), off=torch.from_numpy(off), fine=torch.from_numpy(fine),
                                  k_host=kh)
    return e


def test_wire_round_trip_escape_cpu():
    """Escaped batches travel as version 2 with their shifts and low-bit
    words; batches without an escape stay version 1."""
    e = _fake_batch(seed=4)
    assert int(np.frombuffer(codec.to_bytes(e)[8:12], np.uint32)[0]) == 1
    e = _with_escape(e)
    b = codec.to_bytes(e)
    assert int(np.frombuffer(b[8:12], np.uint32)[0]) == 2
    r = codec.from_bytes(b, device="cpu")
    assert r.escape is not None and np.array_equal(r.escape.k_host, e.escape.k_host)
    ef, rf = e.escape.fine.numpy(), r.escape.fine.numpy()
    for o1, o2, k in zip(e.escape.off.numpy(), r.escape.off.numpy(), e.escape.k_host.reshape(-1)):
        n = 16 * e.nblk * int(k)
        assert np.array_equal(ef[o1:o1 + n], rf[o2:o2 + n])
    assert np.array_equal(r.reference_bytes().numpy(), e.reference_bytes().numpy())
    assert int(r.reference_bytes()[0] - r.reference_bytes()[1]) != 0
    one = r.select(0)
    assert one.escape is not None and one.escape.k_host.shape == (1, 8)


def test_wire_rejects_bad_escape_cpu():
    e = _with_escape(_fake_batch(seed=4))
    e.escape.k_host[0, 1] = 9
    with pytest.raises(codec.WireFormatError, match="escape"):
        codec.from_bytes(codec.to_bytes(e), device="cpu")
    e = _with_escape(_fake_batch(seed=4))
    b = bytearray(codec.to_bytes(e))
    b[8:12] = np.uint32(1).tobytes()   # escape fields in a version-1 batch
    import zlib
    b[-4:] = np.uint32(zlib.crc32(bytes(b[:-4])) & 0xFFFFFFFF).tobytes()
    with pytest.raises(codec.WireFormatError, match="escape"):
        codec.from_bytes(bytes(b), device="cpu")


def _corrupt(field, edit):
    """A fresh valid batch with one field edited (to_bytes writes a valid CRC)."""
    e = _fake_batch(seed=3)
    a = getattr(e, field).clone()
    edit(a)
    setattr(e, field, a)
    return codec.to_bytes(e)


def _set(i, v):
    def f(a):
        a.view(-1)[i] = v
    return f


@pytest.mark.parametrize("field,edit,match", [
    ("blk_n1", _set(0, 7), "coset-1 counts"),                            # count not the bitmap's
    ("coset_bits", lambda a: a.view(-1).__setitem__(5, a.view(-1)[5] ^ 4), "coset-1 counts"),
    ("stream_woff", _set(3, 1), "layout"),                               # a stream moved
    ("stream_nbits", _set(2, 10 ** 6), "layout"),                        # longer than its words
    ("stream_nbits", _set(L.LQ_STREAMS + 9, 64), "bit counts"),          # bits in an absent stream
    ("blk_off", _set(1, 2 ** 30), "checkpoint offsets"),                 # past the stream end
    ("blk_off", _set(0, 5), "checkpoint offsets"),                       # the first block not at bit 0
    ("blk_state", _set(4, 17), "states"),                                # state below L
    ("scale16", lambda a: None, None),                                   # (unchanged: must load)
])
def test_wire_rejects_inconsistent_fields_cpu(field, edit, match):
    b = _corrupt(field, edit)
    if match is None:
        assert codec.from_bytes(b, device="cpu").n_chunks == 2
        return
    with pytest.raises(codec.WireFormatError, match=match):
        codec.from_bytes(b, device="cpu")


def test_wire_rejects_bad_sizes_and_shape_cpu():
    e = _fake_batch(seed=4)
    e.scale16 = e.scale16[:-1].clone()
    with pytest.raises(codec.WireFormatError, match="scale16"):
        codec.from_bytes(codec.to_bytes(e), device="cpu")
    e = _fake_batch(seed=4)
    e.shape = (1, 3, 125, 64)
    with pytest.raises(codec.WireFormatError, match="shape"):
        codec.from_bytes(codec.to_bytes(e), device="cpu")
    e = _fake_batch(seed=4)
    e.blk_n1 = e.blk_n1[:, :-1].clone()
    with pytest.raises(codec.WireFormatError, match="blk_n1"):
        codec.from_bytes(codec.to_bytes(e), device="cpu")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["normal", "outliers", "rotated", "escaped"])
def test_wire_round_trip_decodes_bit_exact_gpu(kind):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3, 1, 4, 256, 128, generator=g)
    if kind == "outliers":
        x[..., :4] *= 10
    if kind == "escaped":   # heavy-tailed K with x20 outlier channels at 5 bits: alphabets beyond L
        rng = np.random.default_rng(7)
        x = torch.from_numpy(rng.standard_t(3.0, size=(3, 1, 4, 1024, 128)).astype(np.float32))
        x[..., [3, 40, 77, 100]] *= 20.0
    x = x.half().cuda()
    if kind == "rotated":
        from latticequant_amd.llm.rotated import decode_rotated, encode_rotated
        enc, _ = encode_rotated(x, 4, [0, 1, 2], [0, 1, 0])
        ref = decode_rotated(enc)
    else:
        enc, _ = codec.encode_batch(x, 5 if kind == "escaped" else 4)
        ref = codec.decode_batch(enc)
        assert (enc.escape is not None) == (kind == "escaped")
    b = codec.to_bytes(enc)
    r = codec.from_bytes(b)
    for a, b2 in zip(_meaningful_tables(enc), _meaningful_tables(r)):
        assert np.array_equal(a, b2)      # rebuilt tables equal the encoder's
    if kind == "rotated":
        from latticequant_amd.llm.rotated import decode_rotated
        got = decode_rotated(r)
    else:
        got = codec.decode_batch(r)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    # the reference-accounted bytes are what the payload carries for them
    assert int(r.reference_bytes().sum()) == int(enc.reference_bytes().sum())


def test_zero_views_layout_cpu():
    """encode_batch's shared zero fill: every part zeroed, 256-byte aligned,
    of its own dtype and size, and disjoint from the others."""
    from latticequant_amd import codec
    st, hist, cwz = codec._zero_views("cpu", (5, torch.int32), (3 * 256, torch.int32), (6, torch.int64))
    assert (st.dtype, hist.dtype, cwz.dtype) == (torch.int32, torch.int32, torch.int64)
    assert (st.numel(), hist.numel(), cwz.numel()) == (5, 768, 6)
    base = st.data_ptr()
    for t in (st, hist, cwz):
        assert (t.data_ptr() - base) % 256 == 0 and int(t.abs().sum()) == 0
    st.fill_(-1)
    hist.fill_(-1)
    assert int(cwz.abs().sum()) == 0   # no overlap
    assert hist.data_ptr() >= st.data_ptr() + 5 * 4 and cwz.data_ptr() >= hist.data_ptr() + 768 * 4
    empty, = codec._zero_views("cpu", (0, torch.int32))
    assert empty.numel() == 0


def test_bits_tensor_cache_cpu():
    """A single int rate gives one cached tensor per (C, rate, device); lists
    are converted per call and checked for length."""
    from latticequant_amd import codec
    a = codec._bits_tensor(4, 3, "cpu")
    assert a is codec._bits_tensor(4, 3, "cpu") and a.tolist() == [4, 4, 4]
    assert codec._bits_tensor(5, 3, "cpu").tolist() == [5, 5, 5]
    assert codec._bits_tensor([3, 4], 2, "cpu").tolist() == [3, 4]
    with pytest.raises(ValueError):
        codec._bits_tensor([3, 4], 3, "cpu")


def test_wire_refuses_other_dither_scheme_cpu(monkeypatch):
    """A batch whose dither seeds stand for another dither scheme is refused
    (its decode would subtract the wrong dither)."""
    e = _fake_batch(seed=6)
    e.extra["dither_seed"] = torch.tensor([11, 12], dtype=torch.int64)
    r = codec.from_bytes(codec.to_bytes(e), device="cpu")
    assert torch.equal(r.extra["dither_seed"], e.extra["dither_seed"])
    monkeypatch.setattr(codec, "DITHER_SCHEME", 1)
    b = codec.to_bytes(e)
    monkeypatch.undo()
    with pytest.raises(codec.WireFormatError, match="dither"):
        codec.from_bytes(b, device="cpu")
