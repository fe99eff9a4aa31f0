"""Rotated + dithered path (the long-context batched workload: seeded per-vector
RHT, subtractive dither, E8 at 4 bits/dim, rANS; batch > 1).

Bit-exact against the oracle on the same inputs: the HeadRHT rotation (fp32,
the reference's butterfly order), the dithered lattice points, every
bitstream word, the in-cache reconstruction and the decoded chunk.  At a
larger shape the round trip is checked through size-independent properties:
the error matches the subtractive-dither theory (per-dimension MSE
G(E8) * scale^2, zero mean, independent of the input)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _oracle_rotate(x, layers, kvs, inverse=False):
    """x: (C, B, H, T, hd) float32 -> HeadRHT of every vector (oracle fp32 transform)."""
    C, B, H, T, hd = x.shape
    out = np.empty_like(x, dtype=np.float32)
    for c in range(C):
        for h in range(H):
            sg = O.rht_signs(hd, O.head_rht_seed(layers[c], h, kvs[c]))
            out[c, :, h] = O.rht_f32(x[c, :, h].reshape(-1, hd), sg, inverse=inverse).reshape(B, T, hd)
    return out


def test_rotated_dithered_vs_oracle_gpu():
    from latticequant_amd import codec
    from latticequant_amd.llm import rotated as R
    g = torch.Generator().manual_seed(17)
    x = torch.randn(2, 2, 3, 64, 128, generator=g).half()
    layers, kvs = [5, 5], [0, 1]
    enc, deq = R.encode_rotated(x.cuda(), 4, layers, kvs, deq_out=True)
    w = _oracle_rotate(x.float().numpy(), layers, kvs)
    s32 = enc.scale32.view(2, -1).cpu().numpy()
    dec = R.decode_rotated(enc).cpu().numpy()
    for c in range(2):
        seed = R.default_dither_seed(layers[c], kvs[c])
        ch = O.compress_chunk(w[c], 4, scales_f32=s32[c], dither_seed=seed)
        base, nw = int(enc.chunk_base[c]), int(enc.chunk_words[c])
        np.testing.assert_array_equal(enc.words[base:base + nw].cpu().numpy().view(np.uint32), ch.bitstream)
        # in-cache reconstruction: ((q - d) * scale32) rotated back, in the input dtype
        want = _oracle_rotate(ch.decompressed[None].astype(np.float32), [layers[c]], [kvs[c]], inverse=True)[0]
        np.testing.assert_array_equal(deq[c].cpu().numpy(), want.astype(np.float16))
        # decode: ((q - d) * scale16) rotated back
        wd = O.decompress_chunk(ch, out_dtype=np.float32)
        want = _oracle_rotate(wd[None], [layers[c]], [kvs[c]], inverse=True)[0]
        np.testing.assert_array_equal(dec[c], want.astype(np.float16))
    # the dither is really on: the same input without it gives different lattice points
    plain, _ = codec.encode_batch(torch.from_numpy(w).cuda(), 4, scale32=enc.scale32)
    assert not torch.equal(plain.words[:int(plain.chunk_words.sum())], enc.words[:int(enc.chunk_words.sum())])


def test_rotated_round_trip_error_statistics_gpu():
    """Batch 8 x 8 heads x 2048 tokens per chunk, 2 chunks: the reconstruction
    error in the rotated domain is the subtractive-dither error times the scale."""
    from latticequant_amd.llm import rotated as R
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(2, 8, 8, 2048, 128, generator=g, device="cuda").half()
    enc, _ = R.encode_rotated(x, 4, [0, 0], [0, 1])
    y = R.decode_rotated(enc, out_dtype=torch.float32)
    e = (y - x.float())
    sc = enc.scale16.float().view(2, 8, 8)                     # (C, B, H) fp16-stored scales
    mse = (e * e).mean(dim=(3, 4)) / (sc * sc)                 # per head, in lattice units
    # G(E8) up to the fp16 rounding of the output (relative 2^-11 on values ~1: adds ~1e-7)
    assert torch.allclose(mse, torch.full_like(mse, R.G_E8), rtol=0.03), mse
    assert e.mean().abs().item() < 2e-3
    # independent of the input
    xf = x.float().flatten()
    ef = e.flatten()
    corr = ((xf - xf.mean()) * (ef - ef.mean())).mean() / (xf.std() * ef.std())
    assert abs(corr.item()) < 0.01
    assert int(enc.status.max()) == 0
