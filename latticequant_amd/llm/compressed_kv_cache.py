"""E8 + rANS compressed KV cache behind HuggingFace's Cache interface
(API of reference llm/compressed_kv_cache.py).

Every update() compresses the new K and V tensors as one chunk each, exactly
as the reference's _compress_tensor does (llm/compressed_kv_cache.py:176-287):
per-head scale sqrt(2 pi e sigma^2 4^-b) (stored fp16), E8 nearest point of
x / scale, symbols (coset bit, 7 free coordinates, floor(c7 / 2)), one rANS
stream per (coset, coordinate) with its own table, coset bits packed
LSB-first.  The bitstreams are the reference's bit for bit.

Differences from the reference, all on the device side:
  * K and V of an update are compressed in one batched launch sequence
    (latticequant_amd.codec) with no host round trip; the chunk's host views
    (streams, stream_meta, coset_counts ...) are materialised only when read.
  * The decompressed K/V handed to attention live in preallocated buffers
    that grow geometrically (amortised O(1) per token instead of torch.cat's
    O(seq) copy, llm/compressed_kv_cache.py:384-395).
  * Side information the decoder uses (per-block checkpoints, compact tables)
    is stored with the chunk and reported by side_info_bytes(); the
    reference-accounted bytes (compressed_bytes()) are the reference's.
  * An uncompressible update (head_dim % 8 != 0) is appended like any other
    (the reference replaces the layer's previous tokens there).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, List, Optional, Tuple

import numpy as np
import torch
from transformers.cache_utils import DynamicCache

from .. import _lib as L
from .. import codec
from ..core.gpu_ans import RANSStream, RANSTable

__all__ = ["pack_coset_bits", "unpack_coset_bits", "OptimizedChunk", "CompressedKVLayer", "UncompressibleKVLayer",
           "CompressedKVCache", "CompressedChunk", "compress_fixed_rate"]


# ------------------------------------------------------- coset bit packing --

def pack_coset_bits(coset: torch.Tensor) -> torch.Tensor:
    """(N,) 0/1 -> ((N+7)//8,) uint8, bit i in byte i//8 at bit i%8
    (llm/compressed_kv_cache.py:46-54)."""
    dev = coset.device
    c = coset.to(torch.uint8)
    if not c.is_cuda:
        c = c.cuda()
    c = c.contiguous()
    n = c.numel()
    out = torch.empty((n + 7) // 8, dtype=torch.uint8, device=c.device)
    L.check(L.lib().lq_pack_coset_bits(c.data_ptr(), n, out.data_ptr(), L.stream_ptr(c.device)), "lq_pack_coset_bits")
    return out if dev.type == "cuda" else out.to(dev)


def unpack_coset_bits(packed: torch.Tensor, n: int) -> torch.Tensor:
    """Inverse of pack_coset_bits -> (n,) uint8 (llm/compressed_kv_cache.py:57-63)."""
    dev = packed.device
    p = packed if packed.is_cuda else packed.cuda()
    p = p.contiguous()
    if p.numel() < (n + 7) // 8:
        raise ValueError("packed holds fewer than n bits")
    out = torch.empty(n, dtype=torch.uint8, device=p.device)
    L.check(L.lib().lq_unpack_coset_bits(p.data_ptr(), n, out.data_ptr(), L.stream_ptr(p.device)),
            "lq_unpack_coset_bits")
    return out if dev.type == "cuda" else out.to(dev)


# ------------------------------------------------------------------ chunk --

class OptimizedChunk:
    """One compressed update of one K or V tensor (llm/compressed_kv_cache.py:69-93).

    Device-resident: the bitstream words, coset bitmap, scales, tables and
    decoder checkpoints stay in the EncodedBatch the chunk was written into.
    The reference's host-side fields are properties materialised on first use."""

    def __init__(self, enc: Optional[codec.EncodedBatch], index: int, scales: torch.Tensor, orig_shape, n_vectors: int,
                 n_heads: int, blocks_per_head: int, bits_per_dim: float, orig_dtype: torch.dtype,
                 pending: Optional[codec.PendingEncode] = None):
        self._enc = enc
        self._index = index
        self._pending = pending
        self._one_raw = enc.select(index) if enc is not None else None
        self.scales = scales
        self.orig_shape = tuple(orig_shape)
        self.n_vectors = n_vectors
        self.n_heads = n_heads
        self.blocks_per_head = blocks_per_head
        self.bits_per_dim = bits_per_dim
        self.orig_dtype = orig_dtype
        self._host = None

    @property
    def _one(self) -> Optional[codec.EncodedBatch]:
        """The chunk's one-chunk batch; a batch written without host syncs is
        settled first (its exact-size arena, or its int16 re-encode)."""
        if self._pending is not None:
            enc = self._pending.result()
            self._enc = enc
            self._one_raw = enc.select(self._index)
            self._host = None
            self._pending = None
        return self._one_raw

    @property
    def encoded(self) -> Optional[codec.EncodedBatch]:
        """The chunk as a one-chunk EncodedBatch (None for eval_only_no_entropy)."""
        return self._one

    def _materialise(self):
        if self._host is None:
            h = {"streams": [], "stream_meta": [], "offsets": [], "counts": (0, 0)}
            if self._one is not None:
                for st in codec.chunk_streams_host(self._one, 0):
                    lo, n_sym = st["lo"], len(st["freqs"])
                    freqs = st["freqs"].astype(np.int32)
                    cum = np.zeros(n_sym + 1, np.int32)
                    cum[1:] = np.cumsum(freqs)
                    lookup = np.repeat(np.arange(n_sym, dtype=np.int32), freqs)
                    tab = RANSTable(lookup=lookup, freqs=freqs, cumfreqs=cum, alphabet=list(range(lo, lo + n_sym)),
                                    n_symbols=n_sym)
                    h["streams"].append(RANSStream(bitstream=st["words"], n_bits=st["n_bits"],
                                                   initial_state=st["state"], n_symbols=st["n"], table=tab))
                    h["stream_meta"].append((st["coset"], st["idx"], st["n"]))
                    h["offsets"].append(st["word_offset"])
                n1 = int(self._one.blk_n1.sum().item())
                h["counts"] = (self.n_vectors - n1, n1)
            self._host = h
        return self._host

    @property
    def streams(self) -> List[RANSStream]:
        return self._materialise()["streams"]

    @property
    def stream_meta(self) -> List[tuple]:
        return self._materialise()["stream_meta"]

    @property
    def stream_word_offsets(self) -> List[int]:
        return self._materialise()["offsets"]

    @property
    def coset_counts(self) -> Tuple[int, int]:
        return self._materialise()["counts"]

    @property
    def gpu_bitstream(self) -> torch.Tensor:
        """(total_words,) int32: the chunk's merged streams."""
        if self._one is None:
            return torch.zeros(1, dtype=torch.int32, device=self.scales.device)
        base = int(self._one.chunk_base[0].item())
        nw = int(self._one.chunk_words[0].item())
        return self._one.words[base:base + nw]

    @property
    def coset_packed(self) -> torch.Tensor:
        """((n_vectors+7)//8,) uint8 coset bitmap."""
        if self._one is None:
            return torch.zeros(1, dtype=torch.uint8, device=self.scales.device)
        return self._one.coset_bits[0, :(self.n_vectors + 7) // 8]

    def reference_bytes(self) -> int:
        """Bytes the reference accounts (llm/compressed_kv_cache.py:113-119)."""
        if self._one is None:
            return 4 + 1 + 2 * self.n_heads
        return int(self._one.reference_bytes()[0].item())

    def side_info_bytes(self) -> int:
        return 0 if self._one is None else int(self._one.side_bytes()[0].item())


class _DeferredGroup:
    """Same-shaped small updates whose entropy coding is batched: their inputs,
    rates and fp32 scales, kept until flush() queues one encode_batch_deferred
    over all of them.  Behaves as the chunks' pending handle: result() flushes
    (if not yet) and settles the batch (a host read of its status and sizes)."""

    def __init__(self):
        self.xs, self.bits, self.scales, self.sigma2, self.chunks = [], [], [], [], []
        self.n = 0
        self._pend = None

    def full(self, limit: int) -> bool:
        return self._pend is not None or self.n >= limit

    def add(self, x: torch.Tensor, bits, scale32: torch.Tensor, sigma2: torch.Tensor) -> int:
        i0 = self.n
        self.xs.append(x)
        self.bits.extend([bits] * x.shape[0] if isinstance(bits, int) else list(bits))
        self.scales.append(scale32)
        self.sigma2.append(sigma2)
        self.n += x.shape[0]
        return i0

    def flush(self) -> Optional[codec.PendingEncode]:
        if self._pend is None and self.n:
            x = self.xs[0] if len(self.xs) == 1 else torch.cat(self.xs)
            bits = self.bits[0] if len(set(self.bits)) == 1 else list(self.bits)
            _, _, self._pend = codec.encode_batch_deferred(x, bits, scale32=torch.cat(self.scales),
                                                          sigma2=torch.cat(self.sigma2))
            self.xs, self.scales, self.sigma2 = [], [], []
            return self._pend
        return None

    @property
    def tracked(self) -> bool:
        return self._pend is not None and self._pend.tracked

    def ready(self) -> bool:
        return self._pend is not None and self._pend.ready()

    def result(self) -> codec.EncodedBatch:
        self.flush()
        return self._pend.result()


class CompressedKVLayer:
    """Chunks of one layer's K or V (llm/compressed_kv_cache.py:96-126)."""

    def __init__(self):
        self.chunks: List[OptimizedChunk] = []

    @property
    def is_empty(self):
        return len(self.chunks) == 0

    @property
    def total_seq(self):
        return sum(c.orig_shape[2] for c in self.chunks) if self.chunks else 0

    @property
    def num_vectors(self):
        return sum(c.n_vectors for c in self.chunks)

    @property
    def total_bytes(self):
        return sum(c.reference_bytes() for c in self.chunks)

    @property
    def side_info_bytes(self):
        return sum(c.side_info_bytes() for c in self.chunks)

    @property
    def fp16_equivalent_bytes(self):
        return self.num_vectors * 8 * 2

    def append_chunk(self, chunk):
        self.chunks.append(chunk)


class UncompressibleKVLayer:
    """Raw storage for head_dim % 8 != 0 (llm/compressed_kv_cache.py:129-143)."""

    def __init__(self, tensor):
        self.data = tensor

    def append(self, tensor):
        self.data = torch.cat([self.data, tensor], dim=2)

    @property
    def is_empty(self):
        return False

    @property
    def total_bytes(self):
        return self.data.nelement() * self.data.element_size()

    @property
    def side_info_bytes(self):
        return 0

    @property
    def fp16_equivalent_bytes(self):
        return self.total_bytes

    @property
    def total_seq(self):
        return self.data.shape[2]


_PLACEHOLDER = None
_PLACEHOLDER_DTYPE = None


def _get_placeholder(device, dtype=torch.bfloat16):
    """Shared empty (1, 1, 0, 1) tensor (llm/compressed_kv_cache.py:146-154)."""
    global _PLACEHOLDER, _PLACEHOLDER_DTYPE
    if _PLACEHOLDER is None or _PLACEHOLDER.device != torch.device(device) or _PLACEHOLDER_DTYPE != dtype:
        _PLACEHOLDER = torch.zeros(1, 1, 0, 1, dtype=dtype, device=device)
        _PLACEHOLDER_DTYPE = dtype
    return _PLACEHOLDER


class _Resident:
    """Growable (B, H, cap, hd) buffer of decompressed tokens; view() is [:, :, :T]."""

    def __init__(self, like: torch.Tensor):
        B, H, T, hd = like.shape
        self.buf = torch.empty((B, H, max(2 * T, 16), hd), dtype=like.dtype, device=like.device)
        self.T = 0

    def append(self, t: torch.Tensor):
        B, H, T, hd = t.shape
        if self.T + T > self.buf.shape[2] or self.buf.shape[0] != B or self.buf.shape[1] != H:
            if self.buf.shape[0] != B or self.buf.shape[1] != H or self.buf.shape[3] != hd:
                raise ValueError("batch / head geometry changed between updates")
            cap = max(2 * self.buf.shape[2], self.T + T)
            nb = torch.empty((B, H, cap, hd), dtype=self.buf.dtype, device=self.buf.device)
            nb[:, :, :self.T].copy_(self.buf[:, :, :self.T])
            self.buf = nb
        self.buf[:, :, self.T:self.T + T].copy_(t)
        self.T += T

    def view(self) -> torch.Tensor:
        return self.buf[:, :, :self.T]

    def nbytes(self) -> int:
        return self.buf[:, :, :self.T].numel() * self.buf.element_size()


# ------------------------------------------------------------------ cache --

class CompressedKVCache(DynamicCache):
    """HF DynamicCache with E8 + rANS compressed storage (llm/compressed_kv_cache.py:161-453)."""

    def __init__(self, bits_per_dim: int = 4, eval_only_no_entropy: bool = False):
        super().__init__()
        assert bits_per_dim in (3, 4, 5)
        self.bits = bits_per_dim
        self.eval_only_no_entropy = eval_only_no_entropy
        self.key_cache: List[torch.Tensor] = []
        self.value_cache: List[torch.Tensor] = []
        self._comp_keys: List[Any] = []
        self._comp_values: List[Any] = []
        self._resident_k: List[Optional[_Resident]] = []
        self._resident_v: List[Optional[_Resident]] = []
        self.total_vectors = 0
        self._model_dtype = None
        self._pending: list = []   # (PendingEncode, chunks) written without host syncs, not yet settled
        self._groups: dict = {}    # (shape, dtype, device) -> open _DeferredGroup of small updates
        self._qscratch = codec.QuantizeScratch()   # small updates' quantizer scratch (the model's stream)
        self._last_layer = -1      # layer of the previous update (a smaller or equal one starts a step)

    # -- compression ----------------------------------------------------
    def _compress_many(self, tensors: List[torch.Tensor], bits=None):
        """Compress same-shaped (B, H, T, hd) tensors in one batched launch.
        Returns [(chunk, decompressed)] in input order.

        Small updates (decode steps) are quantized at once -- the returned K / V
        are final -- while their entropy coding waits in a shared group: once
        DEFER_CHUNKS chunks of one shape are pending (the K and V of every
        layer of a step, typically), or one of them is read, the group is
        encoded in one batch with the scales already computed.  rANS coding is
        lossless and every chunk keeps its own tables and streams, so the
        chunks are the ones a per-update encode writes, with one encode
        launch sequence per group instead of one per update."""
        t0 = tensors[0]
        batch, heads, seq, hd = t0.shape
        if hd % 8 != 0:
            return [("uncompressible", t) for t in tensors]
        bits = self.bits if bits is None else bits
        x = torch.stack([t if t.is_contiguous() else t.contiguous() for t in tensors])
        n_heads = batch * heads
        bph = seq * (hd // 8)
        n_vectors = n_heads * bph
        pend = None
        if not self.eval_only_no_entropy and n_vectors <= self.DEFER_MAX_VECTORS:
            scale32, scale16, deq, sigma2 = codec.quantize_deq(x, bits, self._qscratch)
            key = (tuple(x.shape[1:]), x.dtype, x.device)
            grp = self._groups.get(key)
            if grp is None or grp.full(self.DEFER_CHUNKS):
                if grp is not None:
                    self._flush_group(grp)
                grp = self._groups[key] = _DeferredGroup()
            i0 = grp.add(x, bits, scale32, sigma2)
            per = scale16.view(len(tensors), -1)
            out = []
            for i, t in enumerate(tensors):
                b = bits if isinstance(bits, int) else bits[i]
                ch = OptimizedChunk(None, i0 + i, per[i], t.shape, n_vectors, n_heads, bph, b, t.dtype, pending=grp)
                self.total_vectors += n_vectors
                grp.chunks.append(ch)
                out.append((ch, deq[i]))
            return out
        if self.eval_only_no_entropy:
            _, scale16, deq = codec.quantize_batch(x, bits)
            enc = None
        else:
            # no host sync here: the chunks' status and exact sizes are settled
            # later (_settle_ready at the next update, or on first access)
            enc, deq, pend = codec.encode_batch_deferred(x, bits, deq_out=True)
            scale16 = enc.scale16
        out = []
        per = scale16.view(len(tensors), -1)
        chunks = []
        for i, t in enumerate(tensors):
            b = bits if isinstance(bits, int) else bits[i]
            ch = OptimizedChunk(enc, i, per[i], t.shape, n_vectors, n_heads, bph, b, t.dtype, pending=pend)
            self.total_vectors += n_vectors
            chunks.append(ch)
            out.append((ch, deq[i]))
        if pend is not None:
            self._pending.append((pend, chunks))
        return out

    # small (untracked) pending batches are settled together once this many
    # are pending, or once they keep this many device bytes alive
    SETTLE_SMALL_COUNT = 256
    SETTLE_SMALL_BYTES = 256 << 20
    # updates of at most this many vectors per chunk defer their entropy
    # coding to a shared group of at most DEFER_CHUNKS chunks
    DEFER_MAX_VECTORS = 1 << 14
    DEFER_CHUNKS = 64

    def _flush_group(self, grp: "_DeferredGroup"):
        """Queue the group's batched encode (no host sync) and track it like
        any other pending batch."""
        pend = grp.flush()
        if pend is not None:
            self._pending.append((pend, grp.chunks))

    def _settle_ready(self):
        """Settle the batches whose status read-back has arrived (non-blocking),
        and, once SETTLE_SMALL_COUNT small (untracked) batches are pending or
        they retain SETTLE_SMALL_BYTES of input and arena, all of those with
        one copy: their chunks move to the exact-size arena (or the int16
        re-encode)."""
        small = [p for p, _ in self._pending if not p.tracked]
        if small and (len(small) >= self.SETTLE_SMALL_COUNT
                      or sum(p.retained_bytes() for p in small) >= self.SETTLE_SMALL_BYTES):
            codec.settle_many(small)
        keep = []
        for pend, chunks in self._pending:
            if pend.ready():
                try:
                    for ch in chunks:
                        ch._one   # rebinds the chunk to the settled batch
                except codec.AlphabetError:
                    pass          # the chunks raise it when they are read
            else:
                keep.append((pend, chunks))
        self._pending = keep

    def _compress_tensor(self, tensor: torch.Tensor) -> Tuple[Any, torch.Tensor]:
        """(chunk, decompressed) or ('uncompressible', tensor).  llm/compressed_kv_cache.py:176-287"""
        return self._compress_many([tensor])[0]

    def _decompress_chunk(self, chunk: OptimizedChunk) -> torch.Tensor:
        """rANS decode + dequant with the stored fp16 scales -> orig dtype
        (llm/compressed_kv_cache.py:289-332), in one kernel."""
        if chunk.encoded is None:
            raise ValueError("chunk holds no entropy-coded data (eval_only_no_entropy)")
        out = codec.decode_batch(chunk.encoded, out_dtype=chunk.orig_dtype)
        return out[0]

    def _free_layer(self, layer_idx):
        """Drop a layer's decompressed buffers (llm/compressed_kv_cache.py:334-340)."""
        if layer_idx < len(self.key_cache):
            dev = self.key_cache[layer_idx].device
            dt = self._model_dtype or torch.bfloat16
            self.key_cache[layer_idx] = _get_placeholder(dev, dt)
            self.value_cache[layer_idx] = _get_placeholder(dev, dt)
            self._resident_k[layer_idx] = None
            self._resident_v[layer_idx] = None

    # -- HF Cache interface ----------------------------------------------
    def _layer_bits(self, layer_idx: int):
        return self.bits, self.bits

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None, *args, **kwargs):
        """Compress the new K/V, append, return all K/V of the layer
        (llm/compressed_kv_cache.py:342-395)."""
        device = key_states.device
        if self._model_dtype is None:
            self._model_dtype = key_states.dtype
        # once per step (the layer index stops increasing when a new forward
        # starts): settle the batches whose read-back has arrived
        if layer_idx <= self._last_layer:
            self._settle_ready()
        self._last_layer = layer_idx
        bk, bv = self._layer_bits(layer_idx)
        if key_states.shape == value_states.shape:
            (comp_k, k_new), (comp_v, v_new) = self._compress_many([key_states, value_states],
                                                                   bk if bk == bv else [bk, bv])
        else:
            comp_k, k_new = self._compress_many([key_states], bk)[0]
            comp_v, v_new = self._compress_many([value_states], bv)[0]
        while len(self._comp_keys) <= layer_idx:
            self._comp_keys.append(None)
            self._comp_values.append(None)
            self._resident_k.append(None)
            self._resident_v.append(None)
        while len(self.key_cache) <= layer_idx:
            self.key_cache.append(_get_placeholder(device, self._model_dtype))
            self.value_cache.append(_get_placeholder(device, self._model_dtype))
        if comp_k == "uncompressible":
            if isinstance(self._comp_keys[layer_idx], UncompressibleKVLayer):
                self._comp_keys[layer_idx].append(key_states)
                self._comp_values[layer_idx].append(value_states)
            else:
                self._comp_keys[layer_idx] = UncompressibleKVLayer(key_states)
                self._comp_values[layer_idx] = UncompressibleKVLayer(value_states)
            self.key_cache[layer_idx] = self._comp_keys[layer_idx].data
            self.value_cache[layer_idx] = self._comp_values[layer_idx].data
            return self.key_cache[layer_idx], self.value_cache[layer_idx]
        if self._comp_keys[layer_idx] is None:
            self._comp_keys[layer_idx] = CompressedKVLayer()
            self._comp_values[layer_idx] = CompressedKVLayer()
        self._comp_keys[layer_idx].append_chunk(comp_k)
        self._comp_values[layer_idx].append_chunk(comp_v)
        if self._resident_k[layer_idx] is None:
            self._resident_k[layer_idx] = _Resident(k_new)
            self._resident_v[layer_idx] = _Resident(v_new)
        self._resident_k[layer_idx].append(k_new)
        self._resident_v[layer_idx].append(v_new)
        k_full = self._resident_k[layer_idx].view()
        v_full = self._resident_v[layer_idx].view()
        self.key_cache[layer_idx] = k_full
        self.value_cache[layer_idx] = v_full
        return k_full, v_full

    def get_seq_length(self, layer_idx=0):
        if layer_idx < len(self._comp_keys) and self._comp_keys[layer_idx] is not None:
            return self._comp_keys[layer_idx].total_seq
        return 0

    def get_mask_sizes(self, query_length: int, layer_idx: int = 0) -> tuple:
        """(kv_length, kv_offset) for the attention mask: past tokens + the new query."""
        return self.get_seq_length(layer_idx) + query_length, 0

    def get_max_length(self, layer_idx=None) -> int:
        return -1

    def __len__(self):
        return len(self._comp_keys)

    @property
    def is_compileable(self) -> bool:
        return False

    # -- reporting (llm/compressed_kv_cache.py:399-448) -------------------
    def _layers(self):
        return [x for x in self._comp_keys + self._comp_values if x is not None]

    def compressed_bytes(self):
        return sum(layer.total_bytes for layer in self._layers())

    def side_info_bytes(self):
        """Decoder side information beyond the reference's accounting (checkpoints, tables)."""
        return sum(layer.side_info_bytes for layer in self._layers())

    def fp16_equivalent_bytes(self):
        return sum(layer.fp16_equivalent_bytes for layer in self._layers())

    def decompressed_resident_bytes(self):
        total = 0
        for i in range(len(self.key_cache)):
            for t in (self.key_cache[i], self.value_cache[i]):
                if t is not None:
                    total += t.nelement() * t.element_size()
        return total

    def actual_vram_bytes(self):
        return self.compressed_bytes() + self.decompressed_resident_bytes()

    def memory_report(self):
        comp = self.compressed_bytes()
        fp16 = self.fp16_equivalent_bytes()
        decomp = self.decompressed_resident_bytes()
        actual = self.actual_vram_bytes()
        n_layers = sum(1 for x in self._comp_keys if x is not None)
        eff_bits = (comp * 8) / max(self.total_vectors * 8, 1)
        return "\n".join([
            "CompressedKVCache Report (optimized side info)",
            f"  Bits/dim:     {self.bits} (target), {eff_bits:.3f} (effective)",
            f"  Layers:       {n_layers}",
            f"  Vectors:      {self.total_vectors:,}",
            "  OOR rate:     0.00%",
            "  ---",
            f"  Total compressed:  {comp:,} B ({comp / 1024 / 1024:.2f} MB)",
            f"  Decoder side info: {self.side_info_bytes():,} B",
            f"  Decompressed now:  {decomp:,} B ({decomp / 1024 / 1024:.2f} MB)",
            f"  Actual VRAM (KV):  {actual:,} B ({actual / 1024 / 1024:.2f} MB)",
            f"  FP16 baseline:     {fp16:,} B ({fp16 / 1024 / 1024:.2f} MB)",
            "  ---",
            f"  Theoretical ratio: {fp16 / max(comp, 1):.2f}x",
            f"  Actual ratio:      {fp16 / max(actual, 1):.2f}x",
        ])


# --------------------------------------------------- fixed-rate chunk form --

@dataclass
class CompressedChunk:
    """Fixed-rate chunk (the format llm/fused_triton_merge.py and
    llm/triton_kv_integration.py consume): representable vectors packed at b
    bits/dim, the rest kept as fp16 fallback vectors."""
    repr_mask: torch.Tensor        # (N,) bool, True = packed
    packed: torch.Tensor           # (n_repr, b) uint8
    fallback: torch.Tensor         # (n_oor, 8) fp16: fp16(q * scale) of the out-of-range vectors
    scales: torch.Tensor           # (n_heads,) fp32
    repr_head_ids: torch.Tensor    # (n_repr,) int32 head of each packed vector
    orig_shape: tuple
    n_vectors: int
    n_heads: int
    blocks_per_head: int
    bits_per_dim: int = 4
    orig_dtype: torch.dtype = torch.float16
    # (ceil(N / 1024),) int64 on the device: packed vectors before each
    # 1024-vector tile of repr_mask, when known (compress_fixed_rate sets it;
    # the merge then reads it instead of scanning the mask).  Not stored.
    tile_offsets: Optional[torch.Tensor] = None

    @property
    def total_bytes(self) -> int:
        return (self.packed.numel() + self.fallback.numel() * 2 + (self.n_vectors + 7) // 8
                + self.scales.numel() * self.scales.element_size())


def compress_fixed_rate(tensor: torch.Tensor, bits_per_dim: int = 4, storage_bits: Optional[int] = None,
                        scale32: Optional[torch.Tensor] = None) -> CompressedChunk:
    """Quantize like _compress_tensor (scales at `bits_per_dim`) and store the
    lattice points in the fixed-rate layout at `storage_bits` (default: the
    same), out-of-range vectors as fp16 fallback.  Scales are the fp16-stored
    ones widened to fp32, so merge output equals _decompress_chunk's.  One
    compaction pass on the device (codec.compact_encode); the only host sync
    reads the two row counts that size the chunk's tensors, with the launch's
    look-back error word (codec.LookbackError if it is set)."""
    B, H, T, hd = tensor.shape
    if hd % 8:
        raise ValueError("head_dim must be a multiple of 8")
    x = (tensor.cuda() if not tensor.is_cuda else tensor).contiguous()
    cb = codec.compact_encode(x, bits_per_dim, storage_bits, scale32)
    n_repr, n_oor = codec.compact_counts(cb.totals)
    nh, bph = B * H, T * hd // 8
    return CompressedChunk(repr_mask=cb.mask.view(torch.bool), packed=cb.packed[:n_repr], fallback=cb.fallback[:n_oor],
                           scales=cb.merge_scales, repr_head_ids=cb.repr_heads[:n_repr],
                           orig_shape=(B, H, T, hd), n_vectors=nh * bph, n_heads=nh, blocks_per_head=bph,
                           bits_per_dim=cb.bits, orig_dtype=torch.float16, tile_offsets=cb.tile_off)
