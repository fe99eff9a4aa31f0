"""The benchmark workloads at their own sizes.

C1  [1, 8, 2048, 128] N(0,1) seed 0, 4 bits/dim, no entropy coding: the
    eval-only cache path and the compact 4-bit form (pack -> fused merge),
    bit-exact against the oracle.
C4  Qwen2.5-7B shape [1, 4, 16384, 128] per chunk, K Student-t (nu=3) with 8
    outlier channels x20, V N(0,1), rates cycling 3/4/5: V chunks bit-exact
    against the oracle at full size; each K chunk either round-trips exactly
    (wide path) or raises exactly when an alphabet exceeds L = 1024 symbols,
    decided from the lattice points the device computed.
C5  one full [8, 8, 131072, 128] chunk (2 GiB fp16) through the rotated,
    dithered path: size-independent properties of the round trip (error
    statistics of subtractive dither, status clean, 32-bit stream offsets).
The large cases check properties, not oracle bitstreams, where the oracle
would take minutes."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def test_c1_eval_only_and_compact_gpu():
    from latticequant_amd import codec
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache, compress_fixed_rate
    from latticequant_amd.llm.fused_triton_merge import fused_decompress_chunk
    g = torch.Generator().manual_seed(0)
    k = torch.randn(1, 8, 2048, 128, generator=g).half()
    cache = CompressedKVCache(bits_per_dim=4, eval_only_no_entropy=True)
    kd, _ = cache.update(k.cuda(), k.cuda(), 0)
    q, s32, s16 = codec.quantize_points(k.cuda(), 4)
    s32n = s32.cpu().numpy()
    qo = O.quantize_heads(k.float().numpy(), s32n)
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    want = (qo.reshape(8, -1, 8) * s32n[:, None, None]).astype(np.float32).reshape(k.shape).astype(np.float16)
    np.testing.assert_array_equal(kd.cpu().numpy(), want)
    # fp16 scales from the device sigma^2 agree with the oracle's (torch CPU mean) to the fp16 value
    _, s16o = O.cache_scales(O.head_sigma2(k.float().numpy()), 4)
    np.testing.assert_array_equal(s16.cpu().numpy(), s16o)
    ch = compress_fixed_rate(k.cuda(), bits_per_dim=4)
    mask = O.check_representable(qo, 4)
    np.testing.assert_array_equal(ch.repr_mask.cpu().numpy(), mask)
    np.testing.assert_array_equal(ch.packed.cpu().numpy(), O.pack_e8(qo[mask], 4))
    s16w = ch.scales.cpu().numpy()
    want = (qo.reshape(8, -1, 8) * s16w[:, None, None]).astype(np.float32).astype(np.float16).reshape(k.shape)
    np.testing.assert_array_equal(fused_decompress_chunk(ch).cpu().numpy(), want)


def _student_k(seed, T):
    rng = np.random.default_rng(seed)
    k = rng.standard_t(3.0, size=(1, 4, T, 128)).astype(np.float32)
    for h in range(4):
        k[:, h, :, rng.permutation(128)[:8]] *= 20.0
    return k.astype(np.float16)


@pytest.mark.parametrize("layer", [0, 1, 2])
def test_c4_full_size_layers_gpu(layer):
    """C4 at full size ([1, 4, 16384, 128] per chunk), one layer of the
    3 / 4 / 5-bit cycle per case: V bit-exact against the oracle; K (Student-t
    with outlier channels, int16 symbols) with every stream's table and words
    equal to the oracle's, escaped (coarse streams + raw low bits, equal to the
    oracle's restatement) where an alphabet exceeds L."""
    from latticequant_amd import codec
    from latticequant_amd.allocation.eval_alloc import cyclic_schedule
    from tests.test_wide_gpu import check_chunk, check_escape
    T = 16384
    s = cyclic_schedule(3, seed=0)[layer]
    rng = np.random.default_rng(2026 + layer)
    v = rng.standard_normal((1, 4, T, 128)).astype(np.float16)
    ev, _ = codec.encode_batch(torch.from_numpy(v).cuda()[None], s["V"])
    chv = O.compress_chunk(v, s["V"], scales_f32=ev.scale32.cpu().numpy())
    np.testing.assert_array_equal(ev.words[:int(ev.chunk_words[0])].cpu().numpy().view(np.uint32), chv.bitstream)
    # K: alphabet sizes from the device's own lattice points decide the outcome
    k = _student_k(layer, T)
    kk = torch.from_numpy(k).cuda()
    q, s32, _ = codec.quantize_points(kk, s["K"])
    coset, free, c8h = O.e8_to_symbols(q.cpu().numpy())
    syms = np.concatenate([free, c8h[:, None]], 1)
    widest = max(int(syms[coset == c][:, i].max() - syms[coset == c][:, i].min() + 5)
                 for c in (0, 1) for i in range(8) if (coset == c).any())
    ek, deq = codec.encode_batch(kk[None], s["K"], scale32=s32, deq_out=True)
    assert widest <= 264 or ek.extra["wide"]
    assert (ek.escape is not None) == (widest > O.L)
    want = (q.view(4, -1, 8) * ek.scale16.float().view(4, 1, 1)).view(kk.shape).half()
    assert torch.equal(codec.decode_batch(ek)[0], want)   # lossless coding of the lattice points
    chk = O.compress_chunk(k, s["K"], scales_f32=s32.cpu().numpy(), escape=True)
    widest_coded = check_chunk(ek, 0, chk)
    assert widest_coded == widest if widest <= O.L else widest_coded <= O.L
    check_escape(ek, 0, chk)


def test_c5_full_chunk_round_trip_gpu():
    from latticequant_amd.llm import rotated as R
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(1, 8, 8, 131072, 128, generator=g, device="cuda", dtype=torch.float32).half()
    enc, _ = R.encode_rotated(x, 4, [31], [1], exact_size=False, wide=False)
    assert int(enc.status[0]) == 0
    assert int(enc.stream_nbits.max()) < 2**32
    y = R.decode_rotated(enc)
    e = (y.float() - x.float())
    del y
    sc = enc.scale16.float().view(8, 8)
    mse = (e * e).mean(dim=(3, 4))[0] / (sc * sc)
    assert torch.allclose(mse, torch.full_like(mse, R.G_E8), rtol=0.01), mse
    assert e.mean().abs().item() < 1e-3
    bits_per_dim = 8 * float(enc.reference_bytes().sum()) / x.numel()
    assert 3.3 < bits_per_dim < 4.2, bits_per_dim
