"""End-to-end HF decode over the resident compressed prefix (ResidentKVCache +
the "lq_resident" attention), on a random-init Llama-architecture model.

Each decode step of the model runs lq_resident_attention over the compressed
prefix + fp16 tail.  The reference for the same cache contents is HF's SDPA
over the materialised K / V (prefix dequantised as _decompress_chunk writes
it, then the tail): the same model, teacher-forced with the same tokens, must
give the same next-token logits up to the attention tolerance."""
import pytest
import torch


def _model(seed=0, layers=2, heads=4, kv_heads=2, vocab=512):
    from transformers import LlamaConfig, LlamaForCausalLM
    from latticequant_amd.llm.resident_cache import register
    name = register()
    cfg = LlamaConfig(vocab_size=vocab, hidden_size=heads * 128, intermediate_size=1024, num_hidden_layers=layers,
                      num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=128,
                      max_position_embeddings=4096, attn_implementation=name)
    torch.manual_seed(seed)
    return LlamaForCausalLM(cfg).to(device="cuda", dtype=torch.float16).eval(), cfg


def test_register_and_cache_bookkeeping_cpu():
    from latticequant_amd.llm.resident_cache import ResidentKVCache, register
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    name = register()
    assert name in ALL_ATTENTION_FUNCTIONS.valid_keys()
    c = ResidentKVCache(bits_per_dim=4, tail_tokens=32)
    assert c.get_seq_length() == 0 and c.get_mask_sizes(5) == (5, 0)
    with pytest.raises(ValueError):
        ResidentKVCache(bits_per_dim=6)
    with pytest.raises(ValueError):
        ResidentKVCache(tail_tokens=20)


class _Materialising:
    """Same cache contents, but every update hands HF the materialised K / V."""

    def __init__(self, **kw):
        from latticequant_amd.llm.resident_cache import ResidentKVCache

        class C(ResidentKVCache):
            def update(self, k, v, layer_idx, *a, **kw2):
                super().update(k, v, layer_idx, *a, **kw2)
                return self.materialise(layer_idx)
        self.cache = C(**kw)


@pytest.mark.gpu
@pytest.mark.parametrize("prompt,steps,tail,heads,kv", [(100, 60, 32, 4, 2), (40, 30, 0, 8, 2), (70, 25, 128, 4, 4)])
def test_hf_decode_over_resident_prefix_gpu(prompt, steps, tail, heads, kv, monkeypatch):
    from latticequant_amd.llm.resident_cache import ResidentKVCache
    model, cfg = _model(heads=heads, kv_heads=kv)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, cfg.vocab_size, (1, prompt), generator=g).cuda()
    a = ResidentKVCache(bits_per_dim=4, tail_tokens=tail)
    b = _Materialising(bits_per_dim=4, tail_tokens=tail).cache
    calls = []   # (layer, cache) of every resident-kernel call
    orig = ResidentKVCache.attend
    monkeypatch.setattr(ResidentKVCache, "attend",
                        lambda self, layer, q: calls.append((layer, self)) or orig(self, layer, q))
    with torch.no_grad():
        la = model(ids, past_key_values=a, use_cache=True).logits[:, -1].float()
        lb = model(ids, past_key_values=b, use_cache=True).logits[:, -1].float()
        assert torch.allclose(la, lb)                       # prompt: both take the SDPA path
        agree = 0
        for _ in range(steps):
            nxt = la.argmax(-1, keepdim=True)
            la = model(nxt, past_key_values=a, use_cache=True).logits[:, -1].float()
            lb = model(nxt, past_key_values=b, use_cache=True).logits[:, -1].float()
            # attention agrees to <= 1e-3 relative; two fp16 layers, MLPs and the
            # head carry that into the logits
            err = ((la - lb).abs().max() / lb.abs().max()).item()
            assert err < 5e-3, err
            agree += int(la.argmax() == lb.argmax())
    assert agree >= steps - 1
    # the unmasked decode steps ran the resident kernel in every layer of the
    # cache under test (the materialising cache hands HF plain tensors)
    mine = [layer for layer, c in calls if c is a]
    assert len(mine) == steps * cfg.num_hidden_layers, (len(mine), steps)
    n = prompt + steps
    assert a.get_seq_length() == n == b.get_seq_length()
    flushed = a.res_k[0].n_tokens
    assert flushed % 16 == 0 and n - flushed == a.tail_k[0].shape[2] and a.tail_k[0].shape[2] < tail + 16
    if flushed:
        assert a.compressed_bytes() > 0 and a.resident_bytes() > 0


@pytest.mark.gpu
def test_hf_left_padded_batch_uses_masked_sdpa_gpu(monkeypatch):
    """Batch 2, row 0 left-padded: decode steps carry an attention mask, so the
    "lq_resident" attention must run SDPA over the materialised K / V (pad
    tokens get no weight) and agree with the materialising cache; the
    unmasked kernel path must not run."""
    from latticequant_amd.llm.resident_cache import ResidentKVCache
    model, cfg = _model(heads=4, kv_heads=2)
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, cfg.vocab_size, (2, 48), generator=g).cuda()
    mask = torch.ones(2, 48, dtype=torch.long, device="cuda")
    mask[0, :11] = 0
    a = ResidentKVCache(bits_per_dim=4, tail_tokens=16)
    b = _Materialising(bits_per_dim=4, tail_tokens=16).cache
    calls = []
    orig = ResidentKVCache.attend
    monkeypatch.setattr(ResidentKVCache, "attend", lambda self, layer, q: calls.append(layer) or orig(self, layer, q))
    with torch.no_grad():
        la = model(ids, attention_mask=mask, past_key_values=a, use_cache=True).logits[:, -1].float()
        lb = model(ids, attention_mask=mask, past_key_values=b, use_cache=True).logits[:, -1].float()
        for _ in range(12):
            nxt = la.argmax(-1, keepdim=True)
            mask = torch.cat([mask, torch.ones(2, 1, dtype=mask.dtype, device=mask.device)], 1)
            la = model(nxt, attention_mask=mask, past_key_values=a, use_cache=True).logits[:, -1].float()
            lb = model(nxt, attention_mask=mask, past_key_values=b, use_cache=True).logits[:, -1].float()
            assert torch.equal(la, lb)
    assert calls == []
    assert a.res_k[0].n_tokens > 0   # the prefix was compressed and is read through materialise()


@pytest.mark.gpu
def test_resident_cache_offload_at_rest_gpu():
    """offload_at_rest moves the flushed rANS chunk pairs to host bytes (the
    wire form): decode attention and the materialised K / V are unchanged,
    compressed_bytes is unchanged, the device releases the chunks, and a
    chunk restored from the host decodes to the same K / V the resident prefix
    holds (the values _decompress_chunk writes)."""
    from latticequant_amd import codec
    from latticequant_amd.llm.resident_cache import ResidentKVCache
    g = torch.Generator().manual_seed(5)
    c = ResidentKVCache(bits_per_dim=4, tail_tokens=32)
    k = torch.randn(1, 2, 232, 128, generator=g).half().cuda()
    v = torch.randn(1, 2, 232, 128, generator=g).half().cuda()
    c.update(k[:, :, :200], v[:, :, :200], 0)           # prompt: 160 tokens flushed
    for t in range(200, 232):                           # decode steps: another 32
        c.update(k[:, :, t:t + 1], v[:, :, t:t + 1], 0)
    assert len(c.chunks[0]) == 3 and c.res_k[0].n_tokens == 192
    q = torch.randn(1, 4, 1, 128, generator=g).half().cuda()
    before = c.attend(0, q)
    mk, mv = c.materialise(0)
    ref = c.compressed_bytes()
    torch.cuda.synchronize()
    m0 = torch.cuda.memory_allocated()
    held = c.offload_at_rest()
    torch.cuda.synchronize()
    assert held > 0 and c.at_rest_host_bytes() == held
    assert torch.cuda.memory_allocated() < m0
    assert torch.equal(c.attend(0, q), before)
    mk2, mv2 = c.materialise(0)
    assert torch.equal(mk2, mk) and torch.equal(mv2, mv)
    assert c.compressed_bytes() == ref
    n0 = 160
    for half, full in ((0, mk), (1, mv)):
        dec = codec.decode_batch(c.chunks[0][0][half].batch)
        assert torch.equal(dec.reshape(1, 2, n0, 128), full[:, :, :n0])
    c.restore_at_rest()
    assert c.at_rest_host_bytes() == 0 and c.compressed_bytes() == ref
    assert torch.equal(codec.decode_batch(c.chunks[0][1][0].batch).reshape(1, 2, 16, 128), mk[:, :, n0:n0 + 16])
