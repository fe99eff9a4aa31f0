"""HF cache whose decode steps attend straight over the compressed prefix.

The reference's ``CompressedKVCache.update`` (llm/compressed_kv_cache.py:342-395)
compresses every update and hands HF attention fully decompressed fp16 K / V
(kept resident beside the chunks and ``torch.cat``-ed each step).  Here:

* every layer keeps its newest tokens (up to ``tail_tokens`` + 15) as an fp16
  residual tail; older tokens are flushed in blocks of 16 into
  - E8 + rANS chunks (:func:`codec.encode_batch`, the reference's bitstream
    format: the at-rest form, what ``compressed_bytes`` counts), and
  - the resident fixed-width form of the same lattice points
    (:class:`ResidentKV`) that decode attention reads;
* the at-rest chunks are not read by decode steps: ``offload_at_rest()``
  moves them to host memory in the wire form (the device then keeps the
  resident form and the tail), ``restore_at_rest()`` brings them back;
* ``update`` returns, for a one-token step, marker views that carry the cache
  and layer, and the registered attention ``"lq_resident"`` runs
  ``lq_resident_attention`` over resident prefix + tail (no fp16 prefix is
  ever materialised); for a prompt (several query tokens) it returns the
  materialised K / V (resident prefix dequantised as ``_decompress_chunk``
  writes it, then the tail) for HF's causal SDPA.

Use::

    from latticequant_amd.llm.resident_cache import ResidentKVCache, register
    register()                                   # adds attn_implementation "lq_resident"
    model = AutoModelForCausalLM.from_config(cfg, attn_implementation="lq_resident")
    out = model.generate(ids, past_key_values=ResidentKVCache(bits_per_dim=4), ...)
"""
from __future__ import annotations

from typing import List, Optional

import torch
from transformers.cache_utils import DynamicCache

from .. import codec
from .resident import RB, ResidentKV, attn_workspace, resident_decode_attention

ATTN_NAME = "lq_resident"


class ResidentKVCache(DynamicCache):
    """HF cache: rANS chunks at rest + resident b=5 prefix + fp16 residual tail."""

    def __init__(self, bits_per_dim: int = 4, tail_tokens: int = 128):
        super().__init__()
        if bits_per_dim not in (3, 4, 5):
            raise ValueError("bits_per_dim must be 3, 4 or 5")
        if tail_tokens < 0 or tail_tokens % RB:
            raise ValueError(f"tail_tokens must be a non-negative multiple of {RB}")
        self.bits = bits_per_dim
        self.tail_tokens = tail_tokens
        self.res_k: List[Optional[ResidentKV]] = []
        self.res_v: List[Optional[ResidentKV]] = []
        self.tail_k: List[Optional[torch.Tensor]] = []
        self.tail_v: List[Optional[torch.Tensor]] = []
        self.chunks: List[list] = []          # per layer: [(_AtRest K, _AtRest V)] rANS chunks at rest
        self._work = None
        self._work_heads = 0

    # -- storage ----------------------------------------------------------
    def _ensure(self, layer_idx: int):
        while len(self.res_k) <= layer_idx:
            self.res_k.append(None)
            self.res_v.append(None)
            self.tail_k.append(None)
            self.tail_v.append(None)
            self.chunks.append([])

    def _flush(self, layer_idx: int, n: int):
        """Compress the oldest n (a multiple of 16) tail tokens of the layer."""
        tk, tv = self.tail_k[layer_idx], self.tail_v[layer_idx]
        B, H, _, hd = tk.shape
        xk, xv = tk[:, :, :n].contiguous(), tv[:, :, :n].contiguous()
        # no host sync: the at-rest chunks are settled on first access
        enc, _, pend = codec.encode_batch_deferred(torch.stack([xk, xv]), self.bits)
        s32, s16 = enc.scale32.view(2, -1), enc.scale16.view(2, -1)   # the K and V chunks' head scales
        for i, (res, x) in enumerate(((self.res_k, xk), (self.res_v, xv))):
            r = res[layer_idx]
            if r is None:
                r = ResidentKV(B * H, max(4 * n, 1024), device=x.device)
                res[layer_idx] = r
            elif r.n_tokens + n > r.cap_blocks * RB:
                r.reserve(max(2 * r.cap_blocks * RB, r.n_tokens + n))
            r.append(x, s32[i], s16[i])
        self.chunks[layer_idx].append((_AtRest(pend, 0), _AtRest(pend, 1)))
        self.tail_k[layer_idx] = tk[:, :, n:].contiguous()
        self.tail_v[layer_idx] = tv[:, :, n:].contiguous()

    # -- HF Cache interface ----------------------------------------------
    def update(self, key_states, value_states, layer_idx, cache_kwargs=None, *args, **kwargs):
        if key_states.shape[-1] != 128:
            raise ValueError("ResidentKVCache needs head_dim 128")
        self._ensure(layer_idx)
        if self.tail_k[layer_idx] is None:
            self.tail_k[layer_idx] = key_states.contiguous()
            self.tail_v[layer_idx] = value_states.contiguous()
        else:
            self.tail_k[layer_idx] = torch.cat([self.tail_k[layer_idx], key_states], 2)
            self.tail_v[layer_idx] = torch.cat([self.tail_v[layer_idx], value_states], 2)
        over = self.tail_k[layer_idx].shape[2] - self.tail_tokens
        if over >= RB:
            self._flush(layer_idx, over // RB * RB)
        if key_states.shape[2] == 1:
            # decode step: marker views carrying the cache; the attention reads
            # the resident prefix and the tail itself
            mk, mv = key_states.view_as(key_states), value_states.view_as(value_states)
            mk._lq_cache = mv._lq_cache = self
            mk._lq_layer = mv._lq_layer = layer_idx
            return mk, mv
        return self.materialise(layer_idx)

    def materialise(self, layer_idx: int):
        """Full (B, H, T, hd) K / V of the layer: the resident prefix dequantised
        (lattice point x fp16 scale, rounded once) followed by the tail."""
        tk, tv = self.tail_k[layer_idx], self.tail_v[layer_idx]
        rk, rv = self.res_k[layer_idx], self.res_v[layer_idx]
        if rk is None or rk.n_tokens == 0:
            return tk, tv
        B, H = tk.shape[:2]
        pk = rk.dequant(tk.dtype).view(B, H, -1, 128)
        pv = rv.dequant(tv.dtype).view(B, H, -1, 128)
        return torch.cat([pk, tk], 2), torch.cat([pv, tv], 2)

    def attend(self, layer_idx: int, query: torch.Tensor) -> torch.Tensor:
        """One decode step of the layer: query (B, Hq, 1, 128) -> (B, Hq, 1, 128)."""
        tk, tv = self.tail_k[layer_idx], self.tail_v[layer_idx]
        B, H = tk.shape[:2]
        rk, rv = self.res_k[layer_idx], self.res_v[layer_idx]
        if rk is None:   # nothing flushed yet: an empty prefix
            rk = self.res_k[layer_idx] = ResidentKV(B * H, 1024, device=tk.device)
            rv = self.res_v[layer_idx] = ResidentKV(B * H, 1024, device=tk.device)
        group = query.shape[1] // H
        n = attn_workspace_size(B * H, group, rk.n_tokens, tk.shape[2])
        # the workspace's completion counters sit at [0, 256 * kv heads): a new
        # head count would put split records where counters were, so re-zero
        if (self._work is None or self._work.numel() < n or self._work.device != tk.device or
                self._work_heads != B * H):
            self._work = attn_workspace(B * H, group, rk.n_tokens, tk.shape[2], device=tk.device)
            self._work_heads = B * H
        out = resident_decode_attention(rk, rv, query.to(torch.float16), tk.to(torch.float16),
                                        tv.to(torch.float16), work=self._work)
        return out.to(query.dtype)

    def get_seq_length(self, layer_idx=0):
        if layer_idx >= len(self.tail_k) or self.tail_k[layer_idx] is None:
            return 0
        r = self.res_k[layer_idx]
        return (r.n_tokens if r is not None else 0) + self.tail_k[layer_idx].shape[2]

    def get_mask_sizes(self, query_length: int, layer_idx: int = 0) -> tuple:
        """(kv_length, kv_offset): past tokens + the new query."""
        return self.get_seq_length(layer_idx) + query_length, 0

    def get_max_length(self, layer_idx=None) -> int:
        return -1

    def __len__(self):
        return len(self.tail_k)

    @property
    def is_compileable(self) -> bool:
        return False

    # -- at-rest chunks ---------------------------------------------------
    def offload_at_rest(self) -> int:
        """Move every at-rest chunk pair flushed so far to host memory in the
        wire form (codec.to_bytes: the reference's bitstream words, coset bits
        and fp16 scales plus tables, checkpoints and a CRC-32), releasing its
        device copy: decode steps read only the resident form and the tail, so
        the device then holds about the resident bytes and the tail.  Settles
        pending encodes (one host sync).  Returns the host bytes held."""
        for ch in self.chunks:
            for i, pair in enumerate(ch):
                ch[i] = tuple(e if isinstance(e, _HostAtRest) else _HostAtRest(e.batch) for e in pair)
        return self.at_rest_host_bytes()

    def restore_at_rest(self):
        """Bring offloaded chunk pairs back to the device (codec.from_bytes)."""
        for ch in self.chunks:
            for i, pair in enumerate(ch):
                ch[i] = tuple(_DeviceAtRest(e.batch) if isinstance(e, _HostAtRest) else e for e in pair)

    def at_rest_host_bytes(self) -> int:
        return sum(e.nbytes for ch in self.chunks for pair in ch for e in pair if isinstance(e, _HostAtRest))

    # -- reporting --------------------------------------------------------
    def compressed_bytes(self) -> int:
        """Bytes of the at-rest chunks as the reference counts them
        (bitstream + coset bits + fp16 scales, llm/compressed_kv_cache.py:113-119),
        wherever they are held."""
        return sum(e.reference_bytes() for ch in self.chunks for pair in ch for e in pair)

    def resident_bytes(self) -> int:
        """Bytes of the resident decode form (records, meta, scales, exceptions)."""
        return sum(r.nbytes() for r in self.res_k + self.res_v if r is not None)

    def tail_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.tail_k + self.tail_v if t is not None)


class _AtRest:
    """One K or V half of a flushed chunk pair, settled on first access."""

    def __init__(self, pend, index: int):
        self._pend, self._index = pend, index

    @property
    def batch(self):
        return self._pend.result().select(self._index)

    def reference_bytes(self) -> int:
        return int(self.batch.reference_bytes().sum())


class _DeviceAtRest:
    """An at-rest half held on the device as a settled batch."""

    def __init__(self, batch):
        self.batch = batch

    def reference_bytes(self) -> int:
        return int(self.batch.reference_bytes().sum())


class _HostAtRest:
    """An at-rest half held in host memory in the wire form; .batch restores
    it to the current device (a new device copy per access)."""

    def __init__(self, batch):
        self.blob = codec.to_bytes(batch)
        self.nbytes = len(self.blob)
        self._ref = int(batch.reference_bytes().sum())

    @property
    def batch(self):
        return codec.from_bytes(self.blob)

    def reference_bytes(self) -> int:
        return self._ref


def attn_workspace_size(n_heads: int, group: int, t_prefix: int, t_tail: int) -> int:
    from .. import _lib as L
    n = L.lib().lq_resident_attn_workspace(n_heads, group, t_prefix, t_tail)
    if n < 0:
        raise ValueError("bad attention geometry")
    return int(n)


def resident_attention(module, query, key, value, attention_mask, dropout: float = 0.0, scaling=None, **kwargs):
    """HF attention function "lq_resident": one-token decode steps over a
    ResidentKVCache run lq_resident_attention; everything else (prompts,
    plain tensors) goes to HF's SDPA over the materialised K / V."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    cache = getattr(key, "_lq_cache", None)
    if cache is None or query.shape[2] != 1:
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      **kwargs)
    # The kernel attends to every prefix + tail token with scale 1/sqrt(128).
    # A decode step that needs anything else -- a mask (HF's SDPA mask builder
    # returns None for an unpadded causal step, a tensor e.g. for left-padded
    # batches), a sliding window, logit soft-capping or another scale -- runs
    # SDPA over the materialised K / V instead, as the reference's cache does.
    if (attention_mask is not None or kwargs.get("sliding_window") is not None or
            kwargs.get("softcap") is not None or
            (scaling is not None and abs(scaling - 128 ** -0.5) > 1e-12)):
        k, v = cache.materialise(key._lq_layer)
        return sdpa_attention_forward(module, query, k, v, attention_mask, dropout=dropout, scaling=scaling,
                                      **kwargs)
    out = cache.attend(key._lq_layer, query)            # (B, Hq, 1, hd)
    return out.transpose(1, 2).contiguous(), None        # HF layout (B, q_len, Hq, hd)


def register(name: str = ATTN_NAME) -> str:
    """Register the attention function (and SDPA's mask builder) under `name`."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
    AttentionInterface.register(name, resident_attention)
    AttentionMaskInterface.register(name, sdpa_mask)
    return name
