"""GPU parity of the resident (fixed-width) prefix form and of decode attention over it.

* lq_resident_quantize + lq_resident_dequant: bit-exact with the oracle's
  _decompress_chunk restatement (lattice point times the fp16 scale, rounded
  once), including vectors outside the 5-bit code (exception entries).
* lq_resident_attention: softmax(q K^T / sqrt(128)) V against the oracle in
  float64 over the oracle-dequantised prefix + fp16 tail.  Tolerance (north
  star): 1e-3 relative per query head, max|out - ref| <= 1e-3 * max|ref|.
"""
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


def _data(shape, seed, kind="normal"):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if kind == "outliers":
        x[..., torch.randperm(shape[-1], generator=g)[:4]] *= 10.0
    elif kind == "student":
        d = torch.distributions.StudentT(3.0)
        torch.manual_seed(seed)
        x = d.sample(shape)
        x[..., torch.randperm(shape[-1], generator=g)[:8]] *= 20.0
    return x.half()


def _resident_of(x, bits):
    """Resident prefix + oracle chunk of x (1, H, T, 128), with the oracle's scales."""
    from latticequant_amd.llm.resident import ResidentKV
    ch = O.compress_chunk(x[0].numpy()[None], bits)
    H, T = x.shape[1], x.shape[2]
    r = ResidentKV(H, T, device="cuda")
    r.append(x.cuda(), torch.from_numpy(ch.scales_f32), torch.from_numpy(ch.scales.astype(np.float16)))
    return r, ch


@pytest.mark.parametrize("H,T,bits,kind,seed", [
    (8, 256, 4, "normal", 0),
    (4, 512, 4, "outliers", 1),     # many exceptions (channels x10)
    (2, 160, 3, "normal", 2),
    (2, 160, 5, "normal", 3),
    (4, 64, 3, "student", 4),       # heavy tails: large exception values
])
def test_resident_dequant_bit_exact_gpu(H, T, bits, kind, seed):
    x = _data((1, H, T, 128), seed, kind)
    r, ch = _resident_of(x, bits)
    assert int(r.status.item()) == 0
    got = r.dequant().cpu().numpy()
    ref = O.decompress_chunk(ch).reshape(H, T, 128)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    if kind != "normal":
        assert int(r.n_exc.item()) > 0


def test_resident_append_blocks_and_exception_growth_gpu():
    """Several appends (per-chunk scales), exception list grown on demand."""
    from latticequant_amd.llm.resident import ResidentKV
    xs = [_data((1, 2, 48, 128), 10 + i, "outliers") for i in range(3)]
    r = ResidentKV(2, 144, device="cuda", exc_cap=1)
    refs = []
    for x in xs:
        ch = O.compress_chunk(x[0].numpy()[None], 4)
        r.append(x.cuda(), torch.from_numpy(ch.scales_f32), torch.from_numpy(ch.scales.astype(np.float16)))
        refs.append(O.decompress_chunk(ch).reshape(2, 48, 128))
    assert r.exc_cap >= int(r.n_exc.item()) > 1
    got = r.dequant().cpu().numpy()
    assert np.array_equal(got.view(np.uint16), np.concatenate(refs, 1).view(np.uint16))


def test_resident_matches_chunk_codec_gpu():
    """The resident form holds the lattice points the rANS chunk codes:
    decode_batch (the chunk read path) and the resident dequant agree bit for bit."""
    from latticequant_amd import codec
    from latticequant_amd.llm.resident import from_chunk
    x = _data((1, 8, 1024, 128), 20, "outliers").cuda()
    enc, _ = codec.encode_batch(x[None], 4)
    r = from_chunk(x, enc)
    dec = codec.decode_batch(enc)[0].view(8, 1024, 128)
    assert torch.equal(r.dequant().view(torch.int16), dec.view(torch.int16))


def _attn_case(T_chunks, Hkv, group, tail, seed, bits=4, kind="normal"):
    from latticequant_amd.llm.resident import ResidentKV, resident_decode_attention
    g = torch.Generator().manual_seed(seed + 1000)
    rk = ResidentKV(Hkv, max(16, sum(T_chunks)), device="cuda")
    rv = ResidentKV(Hkv, max(16, sum(T_chunks)), device="cuda")
    ks, vs = [], []
    for i, T in enumerate(T_chunks):
        for r, lst, s in ((rk, ks, 2 * i), (rv, vs, 2 * i + 1)):
            x = _data((1, Hkv, T, 128), seed * 100 + s, kind)
            ch = O.compress_chunk(x[0].numpy()[None], bits)
            r.append(x.cuda(), torch.from_numpy(ch.scales_f32), torch.from_numpy(ch.scales.astype(np.float16)))
            lst.append(O.decompress_chunk(ch).reshape(1, Hkv, T, 128))
    q = torch.randn(1, Hkv * group, 1, 128, generator=g).half()
    tk = torch.randn(1, Hkv, tail, 128, generator=g).half()
    tv = torch.randn(1, Hkv, tail, 128, generator=g).half()
    out = resident_decode_attention(rk, rv, q.cuda(), tk.cuda() if tail else None, tv.cuda() if tail else None)
    K = np.concatenate(ks + [tk.numpy()], 2)
    V = np.concatenate(vs + [tv.numpy()], 2)
    ref = O.decode_attention(q.numpy(), K, V)
    return out.cpu().numpy(), ref


@pytest.mark.parametrize("T_chunks,Hkv,group,tail,seed", [
    ([1024], 8, 4, 128, 0),        # Llama GQA shape, small prefix
    ([512, 1536], 8, 4, 37, 1),    # two chunks (two scales per head), ragged tail
    ([48], 4, 2, 0, 2),            # half tile at the end, no tail
    ([16], 2, 8, 5, 3),            # one block, group 8
    ([512], 4, 1, 1024, 4),        # MHA, long tail (two tail splits)
    ([2048], 4, 7, 64, 5),         # Qwen2.5-7B group 7
    ([96], 1, 16, 3, 6),           # group 16
    ([8192], 2, 16, 40, 8),        # 32 splits x group 16: the final merge takes its records in several batches
])
def test_resident_attention_vs_oracle_gpu(T_chunks, Hkv, group, tail, seed):
    out, ref = _attn_case(T_chunks, Hkv, group, tail, seed)
    assert np.isfinite(out).all()
    assert _rel_err(out, ref) <= 1e-3
    _assert_elementwise(out, ref)


def test_resident_attention_outliers_and_rates_gpu():
    out, ref = _attn_case([1024], 8, 4, 16, 7, kind="outliers")
    assert _rel_err(out, ref) <= 1e-3
    _assert_elementwise(out, ref)
    for b, s in ((3, 8), (5, 9)):
        out, ref = _attn_case([256, 256], 8, 4, 64, s, bits=b)
        assert _rel_err(out, ref) <= 1e-3
        _assert_elementwise(out, ref)


def test_resident_attention_tail_only_gpu():
    from latticequant_amd.llm.resident import ResidentKV, resident_decode_attention
    g = torch.Generator().manual_seed(11)
    rk, rv = ResidentKV(4, 16, device="cuda"), ResidentKV(4, 16, device="cuda")
    q = torch.randn(1, 8, 1, 128, generator=g).half()
    tk = torch.randn(1, 4, 77, 128, generator=g).half()
    tv = torch.randn(1, 4, 77, 128, generator=g).half()
    out = resident_decode_attention(rk, rv, q.cuda(), tk.cuda(), tv.cuda()).cpu().numpy()
    ref = O.decode_attention(q.numpy(), tk.numpy(), tv.numpy())
    assert _rel_err(out, ref) <= 1e-3
    _assert_elementwise(out, ref)


def test_resident_attention_repeat_calls_gpu():
    """The completion counters reset themselves: back-to-back calls on one
    workspace give identical outputs."""
    from latticequant_amd.llm.resident import attn_workspace, from_chunk, resident_decode_attention
    from latticequant_amd import codec
    k = _data((1, 8, 2048, 128), 31).cuda()
    v = _data((1, 8, 2048, 128), 32).cuda()
    ek, _ = codec.encode_batch(k[None], 4)
    ev, _ = codec.encode_batch(v[None], 4)
    rk, rv = from_chunk(k, ek), from_chunk(v, ev)
    q = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(33)).half().cuda()
    work = attn_workspace(8, 4, 2048, 0, device="cuda")
    outs = [resident_decode_attention(rk, rv, q, work=work).clone() for _ in range(4)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    assert int(work[:8 * 256].view(torch.int32).abs().sum()) == 0   # completion counters back at zero


def test_resident_attention_c3_full_size_gpu():
    """C3 shape (32768-token prefix, 8 kv heads, group 4, 128-token tail) against
    float32 attention over the chunk codec's own decoded prefix (the rANS read
    path, itself bit-exact with the oracle at smaller sizes)."""
    from latticequant_amd import codec
    from latticequant_amd.llm.resident import from_chunk, resident_decode_attention
    g = torch.Generator(device="cuda").manual_seed(3)
    k = torch.randn(1, 8, 32768, 128, generator=g, device="cuda").half()
    v = torch.randn(1, 8, 32768, 128, generator=g, device="cuda").half()
    q = torch.randn(1, 32, 1, 128, generator=g, device="cuda").half()
    tk = torch.randn(1, 8, 128, 128, generator=g, device="cuda").half()
    tv = torch.randn(1, 8, 128, 128, generator=g, device="cuda").half()
    ek, _ = codec.encode_batch(k[None], 4)
    ev, _ = codec.encode_batch(v[None], 4)
    rk, rv = from_chunk(k, ek), from_chunk(v, ev)
    Kd = codec.decode_batch(ek)[0].view(8, 32768, 128)
    Vd = codec.decode_batch(ev)[0].view(8, 32768, 128)
    assert torch.equal(rk.dequant().view(torch.int16), Kd.view(torch.int16))
    assert torch.equal(rv.dequant().view(torch.int16), Vd.view(torch.int16))
    out = resident_decode_attention(rk, rv, q, tk, tv).float().view(32, 128)
    K = torch.cat([Kd, tk[0]], 1).float()
    V = torch.cat([Vd, tv[0]], 1).float()
    qf = q.float().view(8, 4, 128)
    s = torch.matmul(qf, K.transpose(1, 2).contiguous()) / 128 ** 0.5
    ref = torch.matmul(torch.softmax(s, -1), V).reshape(32, 128)
    err = ((out - ref).abs().amax(1) / ref.abs().amax(1)).max().item()
    assert err <= 1e-3, err


def test_resident_attention_long_prefix_split_cap_gpu():
    """A prefix long enough that the split count is capped at 2048 / group
    (1 kv head, group 16, 262144 tokens: 128 splits, each wave taking about 8
    tiles) against float32 attention over the resident prefix's own dequantised
    values (bit-exact with the oracle at smaller sizes)."""
    from latticequant_amd import _lib as L
    from latticequant_amd import codec
    from latticequant_amd.llm.resident import from_chunk, resident_decode_attention
    T, G = 262144, 16
    assert L.lib().lq_resident_attn_workspace(1, G, T, 40) > 0
    g = torch.Generator(device="cuda").manual_seed(12)
    k = torch.randn(1, 1, T, 128, generator=g, device="cuda").half()
    v = torch.randn(1, 1, T, 128, generator=g, device="cuda").half()
    q = torch.randn(1, G, 1, 128, generator=g, device="cuda").half()
    tk = torch.randn(1, 1, 40, 128, generator=g, device="cuda").half()
    tv = torch.randn(1, 1, 40, 128, generator=g, device="cuda").half()
    ek, _ = codec.encode_batch(k[None], 4)
    ev, _ = codec.encode_batch(v[None], 4)
    rk, rv = from_chunk(k, ek), from_chunk(v, ev)
    out = resident_decode_attention(rk, rv, q, tk, tv).float().view(G, 128)
    K = torch.cat([rk.dequant().view(T, 128), tk[0, 0]], 0).float()
    V = torch.cat([rv.dequant().view(T, 128), tv[0, 0]], 0).float()
    s = torch.matmul(q.float().view(G, 128), K.t().contiguous()) / 128 ** 0.5
    ref = torch.matmul(torch.softmax(s, -1), V)
    err = ((out - ref).abs().amax(1) / ref.abs().amax(1)).max().item()
    assert err <= 1e-3, err


def test_resident_small_appends_without_host_reads_gpu():
    """Appends of at most ASYNC_MAX_VECTORS vectors read no count back: the
    exception list grows ahead of the host's upper bound of the count (the
    last count read through a pinned copy, plus every vector appended since).
    Many 16-token appends of heavy-tailed data, starting from a one-entry
    list, leave the same records, exception list, scales and dequantised
    values as one large append of the same tokens (which reads the count
    back), and the oracle's values."""
    from latticequant_amd.llm.resident import ResidentKV
    H, n, T = 4, 12, 16
    x = _data((1, H, n * T, 128), 41, "outliers")
    ch = O.compress_chunk(x[0].numpy()[None], 4)
    s32 = torch.from_numpy(ch.scales_f32)
    s16 = torch.from_numpy(ch.scales.astype(np.float16))
    xc = x.cuda()
    small = ResidentKV(H, n * T, device="cuda", exc_cap=1)
    assert H * T * 16 <= small.ASYNC_MAX_VECTORS
    for i in range(n):
        small.append(xc[:, :, i * T:(i + 1) * T], s32, s16)
    big = ResidentKV(H, n * T, device="cuda", exc_cap=1)
    big.ASYNC_MAX_VECTORS = 0   # the read-back path for every append
    big.append(xc, s32, s16)
    torch.cuda.synchronize()
    ne = int(small.n_exc.item())
    assert ne == int(big.n_exc.item()) > 0 and small.exc_cap >= ne
    assert int(small.status.item()) == 0 and int(big.status.item()) == 0
    # records, exception masks and scales are placed per block; the list
    # order of the exceptions (and so the offsets in the meta words) follows
    # the order in which workgroups reserve their slots, so the exceptions are
    # compared through the dequantised values
    for name in ("a", "b", "mask", "scale"):
        assert torch.equal(getattr(small, name), getattr(big, name)), name
    assert torch.equal(small.dequant(), big.dequant())
    got = small.dequant().cpu().numpy()
    ref = O.decompress_chunk(ch).reshape(H, n * T, 128)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
