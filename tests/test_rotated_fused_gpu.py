"""The rotation inside the kernels (lq_head_scales_rht, lq_chunk_quantize_rht,
lq_chunk_decode_rht) against the materialised rotation (lq_rht, then the
plain codec) and the oracle: the same fp32 scales, coset bits and stream
words, and the same decoded rows in every output dtype.  Cases: head_dim
128 / 64 / 32, fp16 and bf16 rows, with and without dither, heads whose vector count is not a
multiple of the 512-vector block (rows and heads cross block boundaries),
heads of fewer than 512 vectors (the quantizer's general launch), and rows
and heads outside the five-operation division's range (IEEE division)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _oracle_rotate(x, layers, kvs, inverse=False):
    C, B, H, T, hd = x.shape
    out = np.empty_like(x, dtype=np.float32)
    for c in range(C):
        for h in range(H):
            sg = O.rht_signs(hd, O.head_rht_seed(layers[c], h, kvs[c]))
            out[c, :, h] = O.rht_f32(x[c, :, h].reshape(-1, hd), sg, inverse=inverse).reshape(B, T, hd)
    return out


CASES = [((2, 2, 3, 64, 128), True), ((1, 2, 2, 40, 128), True), ((2, 1, 4, 96, 64), False),
         ((1, 1, 2, 256, 32), True), ((1, 3, 2, 72, 128), False),
         ((2, 1, 3, 24, 128), True), ((1, 2, 5, 12, 64), False)]   # heads below 512 vectors


@pytest.mark.parametrize("shape,dither,dtype", [(s, d, torch.float16) for s, d in CASES] +
                         [((1, 2, 2, 40, 128), True, torch.bfloat16), ((2, 1, 3, 24, 128), False, torch.bfloat16),
                          ((1, 1, 2, 64, 64), True, torch.bfloat16)])
def test_fused_rotation_matches_materialised_and_oracle_gpu(shape, dither, dtype):
    from latticequant_amd import codec
    from latticequant_amd.llm import rotated as R
    C, B, H, T, hd = shape
    print(f"case {shape} dither={dither} {dtype}", flush=True)
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(T + hd)).to(dtype)
    layers, kvs = list(range(3, 3 + C)), [c & 1 for c in range(C)]
    signs = R.chunk_signs(x.shape, layers, kvs).cuda()
    seeds = [R.default_dither_seed(l, k) for l, k in zip(layers, kvs)] if dither else None
    xc = x.cuda()
    fused, _ = codec.encode_batch(xc, 4, dither_seed=seeds, rht_signs=signs, wide=False)
    w = codec.rotate_rows(xc, signs, inverse=False)
    mat, _ = codec.encode_batch(w, 4, dither_seed=seeds, wide=False)
    assert int(fused.status.max()) == 0
    assert torch.equal(fused.scale32, mat.scale32)
    assert torch.equal(fused.coset_bits, mat.coset_bits)
    assert torch.equal(fused.chunk_words, mat.chunk_words)
    nw = int(fused.chunk_words.sum())
    assert torch.equal(fused.words[:nw], mat.words[:nw])
    # the oracle's rotation and codec on the same scales
    w_or = _oracle_rotate(x.float().numpy(), layers, kvs)
    np.testing.assert_array_equal(w.cpu().numpy(), w_or)
    s32 = fused.scale32.view(C, -1).cpu().numpy()
    for c in range(C):
        ch = O.compress_chunk(w_or[c], 4, scales_f32=s32[c], dither_seed=seeds[c] if dither else None)
        base, n = int(fused.chunk_base[c]), int(fused.chunk_words[c])
        np.testing.assert_array_equal(fused.words[base:base + n].cpu().numpy().view(np.uint32), ch.bitstream)
        if c == 0:
            wd = O.decompress_chunk(ch, out_dtype=np.float32)
            want0 = _oracle_rotate(wd[None], [layers[c]], [kvs[c]], inverse=True)[0].astype(np.float16)
    # decode with the rotation inside the decoder == decode to fp32 + lq_rht inverse
    wd = codec.decode_batch(fused, out_dtype=torch.float32)
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        got = codec.decode_batch(fused, out_dtype=dt, rht_signs=signs)
        want = codec.rotate_rows(wd, signs, inverse=True, out_dtype=dt)
        assert torch.equal(got, want), dt
    np.testing.assert_array_equal(codec.decode_batch(fused, rht_signs=signs)[0].cpu().numpy(), want0)


@pytest.mark.parametrize("dither", [True, False])
def test_fused_rotation_division_fallbacks_gpu(dither):
    """Rotated rows whose values leave [2^-60, 2^60] (zeros, 1e-20, 1e18) and a
    head whose (finite) scale exceeds 2^60 (values ~3e18 at 3 bits: at 4 bits
    every finite scale lies below 2^60) divide by the scale with IEEE division;
    rows in range use the five-operation form.  Both give the materialised
    rotation's words and the oracle's."""
    from latticequant_amd import codec
    from latticequant_amd.llm import rotated as R
    C, B, H, T, hd = 1, 1, 3, 64, 128
    print(f"fallback case dither={dither}", flush=True)
    g = torch.Generator().manual_seed(77)
    x = torch.randn(C, B, H, T, hd, generator=g)
    x[0, 0, 0, 3] = 0.0
    x[0, 0, 0, 5] = 1e-20 * torch.randn(hd, generator=g)
    x[0, 0, 0, 9] = 1e18 * torch.randn(hd, generator=g)
    x[0, 0, 1, 7, :5] = 0.0
    x[0, 0, 2] *= 3e18
    layers, kvs = [4], [1]
    signs = R.chunk_signs(x.shape, layers, kvs).cuda()
    seeds = [R.default_dither_seed(4, 1)] if dither else None
    xc = x.cuda()
    fused, _ = codec.encode_batch(xc, 3, dither_seed=seeds, rht_signs=signs, wide=False)
    w = codec.rotate_rows(xc, signs, inverse=False)
    mat, _ = codec.encode_batch(w, 3, dither_seed=seeds, wide=False)
    s32 = fused.scale32.cpu().numpy()
    assert np.isfinite(s32).all() and s32[2] > 2.0 ** 60 and s32[0] < 2.0 ** 60, s32
    assert int(fused.status.max()) == 0 and int(mat.status.max()) == 0
    assert torch.equal(fused.scale32, mat.scale32)
    assert torch.equal(fused.coset_bits, mat.coset_bits)
    nw = int(fused.chunk_words.sum())
    assert torch.equal(fused.words[:nw], mat.words[:nw])
    w_or = _oracle_rotate(x.numpy(), layers, kvs)
    ch = O.compress_chunk(w_or[0], 3, scales_f32=s32, dither_seed=seeds[0] if dither else None)
    np.testing.assert_array_equal(fused.words[:nw].cpu().numpy().view(np.uint32), ch.bitstream)


def test_encode_decode_rotated_use_fused_path_gpu(monkeypatch):
    """encode_rotated / decode_rotated run the fused entry points (no lq_rht
    launch) unless the reconstruction is asked for."""
    from latticequant_amd import _lib as L
    from latticequant_amd.llm import rotated as R
    lib = L.lib()
    calls = []
    real = lib.lq_rht

    class Spy:
        def __getattr__(self, name):
            if name == "lq_rht":
                def f(*a):
                    calls.append(name)
                    return real(*a)
                return f
            return getattr(lib, name)
    monkeypatch.setattr(L, "lib", lambda: Spy())
    x = torch.randn(1, 2, 2, 64, 128, generator=torch.Generator().manual_seed(9)).half().cuda()
    enc, deq = R.encode_rotated(x, 4, [1], [0])
    y = R.decode_rotated(enc)
    assert deq is None and calls == []
    _, deq = R.encode_rotated(x, 4, [1], [0], deq_out=True)
    assert calls   # the reconstruction path materialises the rotation
    monkeypatch.undo()
    assert torch.equal(R.decode_rotated(enc), y)


@pytest.mark.parametrize("dither", [True, False])
def test_fused_rotation_fp16_extremes_gpu(dither):
    """fp16 rows take the rotation without the division's range test (their
    transform stays on the 2^-24 grid): rows of zeros and negative zeros,
    fp16 subnormals, +-65504 and ordinary rows give the materialised
    rotation's scales, coset bits and words, and the oracle's."""
    from latticequant_amd import codec
    from latticequant_amd.llm import rotated as R
    C, B, H, T, hd = 1, 1, 2, 64, 128
    print(f"fp16 extremes dither={dither}", flush=True)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(C, B, H, T, hd, generator=g)
    x[0, 0, 0, 0] = 0.0
    x[0, 0, 0, 1] = -0.0
    x[0, 0, 0, 2, ::2] = -0.0
    x[0, 0, 0, 3] = 2.0 ** -24
    x[0, 0, 0, 4] = torch.where(torch.arange(hd) % 3 == 0, torch.tensor(-(2.0 ** -24)), torch.tensor(2.0 ** -23))
    x[0, 0, 1, 5] = 65504.0
    x[0, 0, 1, 6] = torch.where(torch.arange(hd) % 2 == 0, torch.tensor(65504.0), torch.tensor(-65504.0))
    x = x.half()
    layers, kvs = [2], [0]
    signs = R.chunk_signs(x.shape, layers, kvs).cuda()
    seeds = [R.default_dither_seed(2, 0)] if dither else None
    xc = x.cuda()
    fused, _ = codec.encode_batch(xc, 4, dither_seed=seeds, rht_signs=signs, wide=False)
    w = codec.rotate_rows(xc, signs, inverse=False)
    mat, _ = codec.encode_batch(w, 4, dither_seed=seeds, wide=False)
    assert int(fused.status.max()) == 0
    assert torch.equal(fused.scale32, mat.scale32)
    assert torch.equal(fused.coset_bits, mat.coset_bits)
    nw = int(fused.chunk_words.sum())
    assert torch.equal(fused.words[:nw], mat.words[:nw])
    w_or = _oracle_rotate(x.float().numpy(), layers, kvs)
    ch = O.compress_chunk(w_or[0], 4, scales_f32=fused.scale32.cpu().numpy(), dither_seed=seeds[0] if dither else None)
    np.testing.assert_array_equal(fused.words[:nw].cpu().numpy().view(np.uint32), ch.bitstream)
