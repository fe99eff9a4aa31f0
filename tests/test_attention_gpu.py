"""GPU parity of the fused compressed decode attention (lq_decode_attention)
against the oracle: K / V dequantised by the oracle's _decompress_chunk
restatement (fp16), tail appended, softmax(q K^T / sqrt(128)) V in float64.

Tolerance (north star): 1e-3 relative, measured per query head against the
largest |output| of that head:  max|out - ref| <= 1e-3 * max|ref| + 1e-4."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _rel_err(out, ref):
    o = out.astype(np.float64).reshape(-1, out.shape[-1])
    r = ref.reshape(-1, ref.shape[-1])
    return (np.abs(o - r).max(1) / (np.abs(r).max(1) + 1e-30)).max()

def _assert_elementwise(out, ref, rtol=1e-3, floor=5e-4, l2=1e-3):
    """Bounds beside the per-head max-norm one (_rel_err): the per-head
    relative error in the 2-norm, ||out - ref|| / ||ref|| <= l2, and every
    output element within rtol of its reference value plus floor x the head's
    largest |ref| (the floor covers entries that cancel to near zero; the fp16
    rounding of the output alone is up to 4.9e-4 relative)."""
    o = out.astype(np.float64).reshape(-1, out.shape[-1])
    r = ref.astype(np.float64).reshape(-1, ref.shape[-1])
    n2 = (np.linalg.norm(o - r, axis=1) / (np.linalg.norm(r, axis=1) + 1e-300)).max()
    lim = rtol * np.abs(r) + floor * np.abs(r).max(1, keepdims=True)
    worst = (np.abs(o - r) / (lim + 1e-300)).max()
    print(f"attention error: 2-norm {n2:.2e}, elementwise {worst:.3f} x the bound")
    assert n2 <= l2, f"per-head relative 2-norm error {n2:.2e}"
    assert worst <= 1.0, f"elementwise error {worst:.3f} x the bound"


def _case(T, n_chunks, Hkv, group, tail, seed, bits=4, outliers=False):
    from latticequant_amd import codec
    from latticequant_amd.llm.decode_attention import decode_attention
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(n_chunks, 1, Hkv, T, 128, generator=g)
    v = torch.randn(n_chunks, 1, Hkv, T, 128, generator=g)
    if outliers:
        k[..., torch.randperm(128, generator=g)[:4]] *= 10.0
    k, v = k.half(), v.half()
    q = torch.randn(1, Hkv * group, 1, 128, generator=g).half()
    tk = torch.randn(1, Hkv, tail, 128, generator=g).half()
    tv = torch.randn(1, Hkv, tail, 128, generator=g).half()
    ek, _ = codec.encode_batch(k.cuda(), bits)
    ev, _ = codec.encode_batch(v.cuda(), bits)
    out = decode_attention(ek, ev, q.cuda(), tk.cuda(), tv.cuda()).cpu().numpy()
    # oracle: dequantised prefix per chunk (bit-exact _decompress_chunk restatement)
    ks, vs = [], []
    for c in range(n_chunks):
        chk = O.compress_chunk(k[c].numpy(), bits, scales_f32=ek.scale32.view(n_chunks, -1)[c].cpu().numpy())
        chv = O.compress_chunk(v[c].numpy(), bits, scales_f32=ev.scale32.view(n_chunks, -1)[c].cpu().numpy())
        ks.append(O.decompress_chunk(chk))
        vs.append(O.decompress_chunk(chv))
    K = np.concatenate(ks + [tk.numpy()], 2)
    V = np.concatenate(vs + [tv.numpy()], 2)
    ref = O.decode_attention(q.numpy(), K, V)
    return out, ref


@pytest.mark.parametrize("T,n_chunks,Hkv,group,tail,seed", [
    (1024, 1, 8, 4, 128, 0),     # Llama GQA, one chunk, whole 32-block workgroups
    (2048, 2, 8, 4, 37, 1),      # two chunks, ragged tail
    (96, 3, 4, 2, 0, 2),         # small chunks (partial workgroups), no tail
    (32, 1, 2, 8, 5, 3),         # one block per head, group 8
    (512, 1, 4, 1, 1024, 4),     # MHA, maximal tail
])
def test_decode_attention_vs_oracle_gpu(T, n_chunks, Hkv, group, tail, seed):
    out, ref = _case(T, n_chunks, Hkv, group, tail, seed)
    assert np.isfinite(out).all()
    assert _rel_err(out, ref) <= 1e-3
    _assert_elementwise(out, ref)


def test_decode_attention_outlier_channels_gpu():
    out, ref = _case(1024, 1, 8, 4, 16, 5, outliers=True)
    assert _rel_err(out, ref) <= 1e-3
    _assert_elementwise(out, ref)


def test_decode_attention_bits_3_5_gpu():
    for b, s in ((3, 6), (5, 7)):
        out, ref = _case(256, 2, 8, 4, 64, s, bits=b)
        assert _rel_err(out, ref) <= 1e-3
        _assert_elementwise(out, ref)


def test_decode_attention_rejects_bad_geometry_gpu():
    from latticequant_amd import codec
    from latticequant_amd.llm.decode_attention import decode_attention
    k = torch.randn(1, 1, 2, 40, 128).half().cuda()
    ek, _ = codec.encode_batch(k, 4)
    with pytest.raises(ValueError):
        decode_attention(ek, ek, torch.randn(1, 2, 1, 128).half().cuda())
    k = torch.randn(1, 1, 2, 32, 64).half().cuda()
    ek, _ = codec.encode_batch(k, 4)
    with pytest.raises(ValueError):
        decode_attention(ek, ek, torch.randn(1, 2, 1, 64).half().cuda())
