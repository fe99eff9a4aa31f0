"""Batched E8 + rANS chunk codec on the GPU (host orchestration of the HIP kernels).

A *chunk* is what one ``CompressedKVCache._compress_tensor`` call produces in
the reference (llm/compressed_kv_cache.py:176-287): a (B, H, T, hd) tensor is
split into n_heads = B*H heads of bph = T*hd/8 eight-dim vectors; each head
gets a per-head scale; vectors are quantized to E8, symbolised (coset bit, 7
free coordinates, floor(c7/2)) and the 16 coordinate streams (2 cosets x 8)
are rANS coded with per-stream tables.

This module keeps a batch of equally shaped chunks resident on the device:

  write:  sigma^2/scales -> quantize (+histograms, coset bitmap, int8 symbols)
          -> tables -> block-parallel encode -> bitstream assembly
  read:   LUT build -> checkpointed decode fused with dequantisation

Nothing here synchronises with the host unless ``exact_size=True`` (the
bitstream arena is then allocated at its exact size) or a host view is asked
for.  All compute runs in the kernels of liblatticequant_amd.so.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from . import _lib as L


def _i(n):
    return int(n)


@dataclass
class EncodedBatch:
    """Device-resident compressed form of n_chunks chunks of one geometry."""
    n_chunks: int
    n_heads: int
    bph: int
    shape: tuple                 # per-chunk (B, H, T, hd)
    bits: torch.Tensor           # (C,) int32
    scale32: torch.Tensor        # (C*H,) fp32, the scale the quantizer divided by
    scale16: torch.Tensor        # (C*H,) fp16, what the chunk stores
    sigma2: Optional[torch.Tensor]
    coset_bits: torch.Tensor     # (C, nblk*BLK/8) uint8, reference LSB-first order
    blk_n1: torch.Tensor         # (C, nblk) int32
    tables: torch.Tensor         # (C*16, TABLE_BYTES) uint8 (lq_table)
    blk_off: torch.Tensor        # (C*16*nblk,) int32 (uint32 bit offsets)
    blk_state: torch.Tensor      # (C*16*nblk,) int16 (uint16 decoder states)
    stream_nbits: torch.Tensor   # (C*16,) int64
    stream_state: torch.Tensor   # (C*16,) int32
    stream_woff: torch.Tensor    # (C*16,) int64 word offset inside the chunk
    chunk_words: torch.Tensor    # (C,) int64
    chunk_base: torch.Tensor     # (C,) int64 word offset of each chunk in `words`
    words: torch.Tensor          # (arena,) int32 merged bitstreams
    status: torch.Tensor         # (C,) int32 LQ_ST_* bits
    hist: Optional[torch.Tensor] = None
    extra: dict = field(default_factory=dict)

    @property
    def n_vectors(self) -> int:
        return self.n_heads * self.bph

    @property
    def nblk(self) -> int:
        return (self.n_vectors + L.LQ_BLK - 1) // L.LQ_BLK

    @property
    def escape(self) -> Optional["Escape"]:
        """Coarse / fine escape of chunks with alphabets beyond L (None: none).
        The wide path plans escapes on the device; the first access reads the
        plan's shifts back (waiting for the plan, not for the whole encode)."""
        esc = self.extra.get("esc")
        if esc is not None and not esc.any():
            self.extra["esc"] = esc = None
        return esc

    # ---- views ------------------------------------------------------------
    def select(self, c: int) -> "EncodedBatch":
        """Chunk c as a one-chunk batch (views, no copies; words stay shared)."""
        C, S, nb = self.n_chunks, L.LQ_STREAMS, self.nblk
        if not 0 <= c < C:
            raise IndexError(c)
        tb = L.TABLE_BYTES
        return EncodedBatch(
            n_chunks=1, n_heads=self.n_heads, bph=self.bph, shape=self.shape, bits=self.bits[c:c + 1],
            scale32=self.scale32.view(C, -1)[c], scale16=self.scale16.view(C, -1)[c],
            sigma2=None if self.sigma2 is None else self.sigma2.view(C, -1)[c],
            coset_bits=self.coset_bits[c:c + 1], blk_n1=self.blk_n1[c:c + 1],
            tables=self.tables[c * S * tb:(c + 1) * S * tb], blk_off=self.blk_off[c * S * nb:(c + 1) * S * nb],
            blk_state=self.blk_state[c * S * nb:(c + 1) * S * nb], stream_nbits=self.stream_nbits[c * S:(c + 1) * S],
            stream_state=self.stream_state[c * S:(c + 1) * S], stream_woff=self.stream_woff[c * S:(c + 1) * S],
            chunk_words=self.chunk_words[c:c + 1], chunk_base=self.chunk_base[c:c + 1], words=self.words,
            status=self.status[c:c + 1],
            hist=None if self.hist is None else self.hist.view(C, -1)[c],
            extra={**self.extra, "dither_seed": None if self.extra.get("dither_seed") is None
                   else self.extra["dither_seed"][c:c + 1],
                   "esc": None if self.escape is None else self.escape.select(c)})

    # ---- byte accounting -------------------------------------------------
    def reference_bytes(self) -> torch.Tensor:
        """Bytes the reference counts per chunk (llm/compressed_kv_cache.py:113-119):
        int32 bitstream words + packed coset bits + fp16 scales, plus, for an
        escaped chunk (alphabets beyond L, a case the reference never
        completes), its raw low-bit words.  (C,) int64 on device."""
        b = self.chunk_words * 4 + (self.n_vectors + 7) // 8 + 2 * self.n_heads
        if self.escape is not None:
            b = b + self.escape.fine_bytes(self.nblk).to(b.device)
        return b

    def side_bytes(self) -> torch.Tensor:
        """Bytes this format adds per chunk: compact tables (lo, n_sym: 4 B + 2 B per
        symbol), block checkpoints (4 B offset + 2 B state per stream and block),
        per-block coset counts (2 B)."""
        t = self.tables.view(torch.int32).view(-1, L.TABLE_BYTES // 4)
        nsym = t[:, 1].to(torch.int64).view(self.n_chunks, L.LQ_STREAMS)
        present = (nsym > 0).to(torch.int64)
        tab = (4 * present + 2 * nsym).sum(1)
        ck = 6 * present.sum(1) * self.nblk
        return tab + ck + 2 * self.nblk


class Escape:
    """Coarse / fine escape of a batch (lq_chunk_escape_plan / _split): per
    chunk and coordinate j the shift k_j; symbol s of coordinate j is coded as
    s >> k_j in its stream and its k_j low bits are stored raw in `fine`
    (coordinate j of chunk c: nblk * 16 * k_j words from word off[c * 8 + j],
    vector v's bits at bit v * k_j, least significant first).  A format of this
    build: the reference never terminates on alphabets beyond L.

    k: (C, 8) int32, device; off: (C * 8,) int64 word offsets into fine,
    device; fine: int32 words, device (one slack word past the last).  A plan
    made on the device (`pending`: the pinned copy of the shifts, the event
    after it, the stream that wrote `fine`, nblk) keeps `fine` at its upper
    bound until k_host is first read; then a batch with escapes keeps only its
    words (copied on the writing stream, so after the split that fills them)."""

    def __init__(self, k: torch.Tensor, off: torch.Tensor, fine: torch.Tensor,
                 k_host: Optional[np.ndarray] = None, pending=None):
        self.k, self.off, self.fine = k, off, fine
        self._k_host = k_host
        self._pending = pending
        if k_host is None and pending is None:
            raise ValueError("Escape needs the host shifts or a pending device plan")

    @property
    def k_host(self) -> np.ndarray:
        """(C, 8) int32 shifts on the host."""
        if self._k_host is None:
            host, event, stream, nblk = self._pending
            event.synchronize()
            kh = host.numpy().reshape(-1, 8).astype(np.int32)
            total = int((16 * nblk * kh.astype(np.int64)).sum())
            if total and total + 1 < self.fine.numel():
                with torch.cuda.stream(stream):
                    self.fine = self.fine[:total + 1].clone()
            self._k_host, self._pending = kh, None
        return self._k_host

    def any(self) -> bool:
        return bool(self.k_host.any())

    def ready(self) -> bool:
        """The shifts are on the host, or their copy has arrived (non-blocking)."""
        return self._pending is None or self._pending[1].query()

    def select(self, c: int) -> "Escape":
        kh = self.k_host[c:c + 1]   # first: reading the plan may compact fine
        return Escape(k=self.k[c:c + 1], off=self.off[8 * c:8 * c + 8], fine=self.fine, k_host=kh)

    def fine_bytes(self, nblk: int) -> torch.Tensor:
        """Raw low-bit bytes per chunk, (C,) int64 (host tensor)."""
        return torch.from_numpy(4 * 16 * nblk * self.k_host.astype(np.int64).sum(1))


def _plan_escape(minmax, C, nblk, V, sym, coset_bits, blk_n1, status, dev, s):
    """Escape plan and split of a wide batch, with no host read: the fine-word
    offsets are an exclusive scan of 16 nblk k_j on the device, the fine
    buffer has its upper bound (k_j <= LQ_ESC_MAX_SHIFT), and the shifts
    reach the host through a pinned copy that Escape.k_host waits for.
    Returns (Escape, the coarse per-stream min / max)."""
    lib = L.lib()
    esc_k = _empty(C * 8, torch.int32, dev)
    mm_c = torch.empty_like(minmax)
    L.check(lib.lq_chunk_escape_plan(minmax.data_ptr(), C, esc_k.data_ptr(), mm_c.data_ptr(), status.data_ptr(), s),
            "lq_chunk_escape_plan")
    stream = torch.cuda.current_stream(dev)
    host = torch.empty(C * 8, dtype=torch.int32, pin_memory=True)
    host.copy_(esc_k, non_blocking=True)
    event = torch.cuda.Event()
    event.record(stream)
    per = esc_k.to(torch.int64) * (16 * nblk)
    off_d = torch.cumsum(per, 0) - per
    fine = _empty(C * 8 * 16 * nblk * L.LQ_ESC_MAX_SHIFT + 1, torch.int32, dev)
    L.check(lib.lq_chunk_escape_split(sym.data_ptr(), coset_bits.data_ptr(), blk_n1.data_ptr(), C, V, esc_k.data_ptr(),
                                      off_d.data_ptr(), fine.data_ptr(), s), "lq_chunk_escape_split")
    return Escape(k=esc_k.view(C, 8), off=off_d, fine=fine, pending=(host, event, stream, nblk)), mm_c


def words_bound(n_chunks: int, n_vectors: int) -> int:
    """Upper bound of the bitstream words of n_chunks chunks (10 bits per symbol,
    n_words + 1 per stream) plus the decoder's 2-word read-ahead slack."""
    return n_chunks * ((10 * 8 * n_vectors + 31) // 32 + 2 * L.LQ_STREAMS) + 2


def _zeros(n, dtype, dev):
    return torch.zeros(int(n), dtype=dtype, device=dev)


def _empty(n, dtype, dev):
    return torch.empty(int(n), dtype=dtype, device=dev)


def _zero_views(dev, *parts):
    """Zeroed device arrays, one per (n, dtype) part, cut from one buffer
    cleared by one fill; each starts 256-byte aligned."""
    sizes = [int(n) * torch.empty((), dtype=dt).element_size() for n, dt in parts]
    offs, total = [], 0
    for nb in sizes:
        offs.append(total)
        total += (nb + 255) // 256 * 256
    z = torch.zeros(max(total, 256), dtype=torch.uint8, device=dev)
    return [z[o:o + nb].view(dt) for (_, dt), o, nb in zip(parts, offs, sizes)]


_BITS_CACHE = {}


def _bits_tensor(bits, C, dev):
    """Per-chunk rates on the device.  A single int rate gives a cached
    read-only tensor per (C, rate, device), so a steady stream of same-shaped
    batches launches no fill for it.  Kernels on any stream may read a cached
    entry: its fill is complete before it is first returned (one stream
    synchronisation per entry), and entries are never freed while the process
    runs; past 256 entries a new shape gets a per-call tensor, which only the
    current stream reads."""
    if isinstance(bits, int):
        key = (int(C), int(bits), torch.device(dev))
        t = _BITS_CACHE.get(key)
        if t is None:
            t = torch.full((C,), bits, dtype=torch.int32, device=dev)
            if len(_BITS_CACHE) < 256:
                if t.is_cuda:
                    torch.cuda.current_stream(t.device).synchronize()
                _BITS_CACHE[key] = t
        return t
    b = torch.as_tensor(list(bits), dtype=torch.int32)
    if b.numel() != C:
        raise ValueError("bits must be an int or one value per chunk")
    return b.to(dev)


def _head_scales(x: torch.Tensor, bits, scale32: Optional[torch.Tensor], rht_signs: Optional[torch.Tensor] = None):
    """Per-head scales of a (C, B, H, T, hd) batch: from sigma^2 on the device
    (llm/compressed_kv_cache.py:188-196) or the caller's fp32 scales, plus the
    fast-division flags of the quantizer.  rht_signs: sigma^2 of the rows
    rotated in the kernel (the flags are then 0: rotated values are fp32)."""
    lib = L.lib()
    C, B, H, T, hd = x.shape
    dev = x.device
    nh, bph = B * H, T * hd // 8
    dt = L.dtype_code(x.dtype)
    s = L.stream_ptr(dev)
    bits_t = _bits_tensor(bits, C, dev)
    fastdiv = _empty(C * nh, torch.int32, dev)
    sigma2 = None
    if scale32 is None:
        work = _empty(4096 + C * nh, torch.float64, dev)
        sigma2 = _empty(C * nh, torch.float32, dev)
        scale32 = _empty(C * nh, torch.float32, dev)
        scale16 = _empty(C * nh, torch.float16, dev)
        if rht_signs is not None:
            L.check(lib.lq_head_scales_rht(x.data_ptr(), dt, C, nh, bph, hd, rht_signs.data_ptr(), bits_t.data_ptr(),
                                           work.data_ptr(), sigma2.data_ptr(), scale32.data_ptr(), scale16.data_ptr(),
                                           fastdiv.data_ptr(), s), "lq_head_scales_rht")
        else:
            L.check(lib.lq_head_scales(x.data_ptr(), dt, C, nh, bph, bits_t.data_ptr(), work.data_ptr(),
                                       sigma2.data_ptr(), scale32.data_ptr(), scale16.data_ptr(), fastdiv.data_ptr(), s),
                    "lq_head_scales")
    else:
        scale32 = scale32.to(device=dev, dtype=torch.float32).contiguous().view(-1)
        if scale32.numel() != C * nh:
            raise ValueError("scale32 must hold one scale per head of every chunk")
        scale16 = scale32.to(torch.float16)
        fd_dt = L.LQ_F32 if rht_signs is not None else dt
        L.check(lib.lq_scale_fastdiv(scale32.data_ptr(), C * nh, fd_dt, fastdiv.data_ptr(), s), "lq_scale_fastdiv")
    return bits_t, scale32, scale16, sigma2, fastdiv


def _check_signs(signs: torch.Tensor, rows: int, hd: int, dev) -> torch.Tensor:
    """RHT sign rows as the kernels read them: (rows, hd) fp32 on the device."""
    if hd < 8 or hd > 512 or hd & (hd - 1):
        raise ValueError(f"the rotation needs a power-of-two head_dim in [8, 512], got {hd}")
    sg = signs.to(device=dev, dtype=torch.float32).contiguous()
    if sg.numel() != rows * hd:
        raise ValueError(f"rht_signs must hold {rows} rows of {hd} signs")
    return sg.view(rows, hd)


def rotate_rows(x: torch.Tensor, signs: torch.Tensor, inverse: bool, out_dtype=torch.float32) -> torch.Tensor:
    """RHT of every hd-row of a (C, B, H, T, hd) batch, row (c*B + b)*H + h of
    `signs` for head (c, b, h) (lq_rht; fp32 arithmetic)."""
    lib = L.lib()
    C, B, H, T, hd = x.shape
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    L.check(lib.lq_rht(x.data_ptr(), L.dtype_code(x.dtype), x.numel() // hd, hd, signs.data_ptr(), T,
                       signs.shape[0], 1 if inverse else 0, out.data_ptr(), L.dtype_code(out_dtype),
                       L.stream_ptr(x.device)), "lq_rht")
    return out


def _check_input(x: torch.Tensor) -> torch.Tensor:
    if x.dim() != 5:
        raise ValueError("x must be (n_chunks, B, H, T, hd)")
    if not x.is_cuda:
        raise ValueError("x must be a CUDA (ROCm) tensor")
    if x.shape[-1] % 8:
        raise ValueError("head_dim must be a multiple of 8")
    if x.numel() == 0:
        raise ValueError("empty chunk")
    return x.contiguous()


def quantize_batch(x: torch.Tensor, bits, scale32: Optional[torch.Tensor] = None, with_sigma2: bool = False):
    """E8-quantize a batch of chunks without entropy coding (the reference's
    eval_only_no_entropy path, llm/compressed_kv_cache.py:199-221).
    Returns (scale32, scale16, deq) with deq = q * scale32 in x's dtype, and
    sigma2 after them when with_sigma2 (None for caller scales)."""
    lib = L.lib()
    x = _check_input(x)
    C, B, H, T, hd = x.shape
    dev = x.device
    nh, bph = B * H, T * hd // 8
    nblk = (nh * bph + L.LQ_BLK - 1) // L.LQ_BLK
    dt = L.dtype_code(x.dtype)
    _, scale32, scale16, sigma2, fastdiv = _head_scales(x, bits, scale32)
    sym = _empty(C * nblk * L.LQ_SYM_STRIDE, torch.int8, dev)
    coset_bits = _empty(C * nblk * L.LQ_BLK // 8, torch.uint8, dev)
    blk_n1 = _empty(C * nblk, torch.int32, dev)
    status, hist = _zero_views(dev, (C, torch.int32), (C * L.LQ_STREAMS * 256, torch.int32))
    deq = torch.empty_like(x)
    L.check(lib.lq_chunk_quantize(x.data_ptr(), dt, C, nh, bph, scale32.data_ptr(), fastdiv.data_ptr(), sym.data_ptr(),
                                  coset_bits.data_ptr(), blk_n1.data_ptr(), hist.data_ptr(), status.data_ptr(),
                                  deq.data_ptr(), dt, None, L.stream_ptr(dev)), "lq_chunk_quantize")
    return (scale32, scale16, deq, sigma2) if with_sigma2 else (scale32, scale16, deq)


class QuantizeScratch:
    """Device scratch of quantize_deq, grown on demand and reused: calls that
    share one must run on one stream (in order)."""

    def __init__(self):
        self.buf: Optional[torch.Tensor] = None

    def get(self, C: int, nh: int, bph: int, dev) -> torch.Tensor:
        n = int(L.lib().lq_quantize_deq_workspace(C, nh, bph))
        if n < 0:
            raise ValueError("invalid chunk geometry")
        b = self.buf
        if b is None or b.device != torch.device(dev) or b.numel() < n:
            self.buf = b = torch.empty(max(n, 2 * b.numel() if b is not None else 0), dtype=torch.uint8, device=dev)
        return b


def quantize_deq(x: torch.Tensor, bits, scratch: QuantizeScratch):
    """quantize_batch(x, bits, with_sigma2=True) in one native call
    (lq_quantize_deq): (scale32, scale16, deq, sigma2), with the symbol
    staging and the other by-products in the caller's scratch, so a decode
    step's update allocates only its outputs."""
    lib = L.lib()
    x = _check_input(x)
    C, B, H, T, hd = x.shape
    dev = x.device
    nh, bph = B * H, T * hd // 8
    work = scratch.get(C, nh, bph, dev)
    n = C * nh
    sc = torch.empty(3 * n, dtype=torch.float32, device=dev)   # sigma2 | scale32 | scale16 (fp16, front half)
    sigma2, scale32 = sc[:n], sc[n:2 * n]
    scale16 = sc[2 * n:].view(torch.float16)[:n]
    deq = torch.empty_like(x)
    bits_t = _bits_tensor(bits, C, dev)
    L.check(lib.lq_quantize_deq(x.data_ptr(), L.dtype_code(x.dtype), C, nh, bph, bits_t.data_ptr(), work.data_ptr(),
                                sigma2.data_ptr(), scale32.data_ptr(), scale16.data_ptr(), deq.data_ptr(),
                                L.stream_ptr(dev)), "lq_quantize_deq")
    return scale32, scale16, deq, sigma2


def quantize_points(t: torch.Tensor, bits, scale32: Optional[torch.Tensor] = None):
    """Lattice points of one (B, H, T, hd) tensor as _compress_tensor computes
    them (x / scale[head] -> E8).  Returns (q (B*H*T*hd/8, 8) fp32, scale32, scale16)."""
    lib = L.lib()
    x = _check_input(t[None])
    _, B, H, T, hd = x.shape
    nh, bph = B * H, T * hd // 8
    _, scale32, scale16, _, fastdiv = _head_scales(x, bits, scale32)
    q = torch.empty(nh * bph, 8, dtype=torch.float32, device=x.device)
    L.check(lib.lq_e8_quantize_heads(x.data_ptr(), L.dtype_code(x.dtype), nh, bph, scale32.data_ptr(), fastdiv.data_ptr(),
                                     q.data_ptr(), L.stream_ptr(x.device)), "lq_e8_quantize_heads")
    return q, scale32, scale16


@dataclass
class CompactBatch:
    """Device output of compact_encode: the fixed-rate form of one tensor with
    buffers sized for every vector (packed / fallback rows beyond the totals
    are unused) and the counts still on the device."""
    mask: torch.Tensor         # (V,) uint8, 1 = packed
    packed: torch.Tensor       # (V, bits) uint8; rows < totals[0] hold the packed points
    fallback: torch.Tensor     # (V, 8) fp16; rows < totals[1] hold the out-of-range vectors
    repr_heads: torch.Tensor   # (V,) int32; rows < totals[0]: head of each packed point
    tile_off: torch.Tensor     # (tiles,) int64: packed points before each 1024-vector tile
    totals: torch.Tensor       # (3,) int64: (n_packed, n_fallback, look-back error word)
    scale32: torch.Tensor      # (n_heads,) fp32 quantization scales
    scale16: torch.Tensor      # (n_heads,) fp16 stored scales
    shape: tuple
    bph: int
    bits: int
    merge_scales: Optional[torch.Tensor] = None   # (n_heads,) fp32: float(scale16), the merge's scales


def compact_encode(t: torch.Tensor, bits: int, storage_bits: Optional[int] = None,
                   scale32: Optional[torch.Tensor] = None) -> CompactBatch:
    """Fixed-rate compression of one (B, H, T, hd) tensor without a host sync:
    scales at `bits` (or the caller's scale32), lattice points packed at
    `storage_bits` (default `bits`) where they fit, fp16 fallback elsewhere,
    compacted in one pass.  Device scales with T * hd / 8 >= 1024 vectors per
    head: two launches (lq_compact_encode_scaled finalises the scales inside
    the encoder); otherwise lq_head_scales (or lq_scale_fastdiv) and
    lq_compact_encode."""
    lib = L.lib()
    sb = storage_bits or bits
    if sb not in (3, 4, 5):
        raise ValueError("storage bits must be 3, 4 or 5")
    x = _check_input(t[None])
    _, B, H, T, hd = x.shape
    nh, bph = B * H, T * hd // 8
    V = nh * bph
    dev = x.device
    tiles = (V + 1023) // 1024
    mask = _empty(V, torch.uint8, dev)
    packed = _empty(V * sb, torch.uint8, dev).view(V, sb)
    fallback = _empty(V * 8, torch.float16, dev).view(V, 8)
    heads = _empty(V, torch.int32, dev)
    tile_off = _empty(tiles, torch.int64, dev)
    totals = _empty(3, torch.int64, dev)
    st = L.stream_ptr(dev)
    if scale32 is None and bph >= 1024 and isinstance(bits, int):
        scale32 = _empty(nh, torch.float32, dev)
        scale16 = _empty(nh, torch.float16, dev)
        merge_scales = _empty(nh, torch.float32, dev)
        work = _empty(lib.lq_compact_encode_scaled_workspace(nh, bph), torch.uint8, dev)
        L.check(lib.lq_compact_encode_scaled(x.data_ptr(), L.dtype_code(x.dtype), nh, bph, bits, sb, None,
                                             scale32.data_ptr(), scale16.data_ptr(), merge_scales.data_ptr(),
                                             mask.data_ptr(), packed.data_ptr(), fallback.data_ptr(), heads.data_ptr(),
                                             tile_off.data_ptr(), totals.data_ptr(), work.data_ptr(), st),
                "lq_compact_encode_scaled")
    else:
        _, scale32, scale16, _, fastdiv = _head_scales(x, bits, scale32)
        work = _empty(lib.lq_compact_encode_workspace(V), torch.uint8, dev)
        L.check(lib.lq_compact_encode(x.data_ptr(), L.dtype_code(x.dtype), nh, bph, scale32.data_ptr(),
                                      fastdiv.data_ptr(), scale16.data_ptr(), sb, mask.data_ptr(), packed.data_ptr(),
                                      fallback.data_ptr(), heads.data_ptr(), tile_off.data_ptr(), totals.data_ptr(),
                                      work.data_ptr(), st), "lq_compact_encode")
        merge_scales = scale16.float()
    return CompactBatch(mask=mask, packed=packed, fallback=fallback, repr_heads=heads, tile_off=tile_off,
                        totals=totals, scale32=scale32, scale16=scale16, shape=(B, H, T, hd), bph=bph, bits=sb,
                        merge_scales=merge_scales)


class LookbackError(RuntimeError):
    """A chained look-back wait did not end within its spin limit: the ranks,
    offsets and totals of that launch are invalid."""


def compact_counts(totals) -> tuple:
    """(n_packed, n_fallback) from a CompactBatch's totals, read to the host in
    one copy; raises LookbackError when the launch set its error word."""
    n_repr, n_oor, err = (int(v) for v in totals.tolist())
    if err:
        raise LookbackError("lq_compact_encode: a tile look-back wait did not end; the batch is invalid")
    return n_repr, n_oor


def compact_merge(cb: CompactBatch, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp16 (B, H, T, hd) from a CompactBatch (lq_compact_merge: packed points
    dequantised with float(scale16), fallback rows copied), no host sync."""
    lib = L.lib()
    B, H, T, hd = cb.shape
    V = cb.mask.numel()
    dev = cb.mask.device
    if out is None:
        out = torch.empty(B, H, T, hd, dtype=torch.float16, device=dev)
    sc = cb.merge_scales if cb.merge_scales is not None else cb.scale16.float()
    L.check(lib.lq_compact_merge(cb.packed.data_ptr(), V, cb.bits, cb.fallback.data_ptr(), V, cb.mask.data_ptr(),
                                 sc.data_ptr(), V, cb.bph, cb.tile_off.data_ptr(), out.data_ptr(), L.stream_ptr(dev)),
            "lq_compact_merge")
    return out


def _status_or(status: torch.Tensor) -> int:
    """OR of the per-chunk LQ_ST_* bits (one device-to-host copy)."""
    st = 0
    for v in status.cpu().tolist():
        st |= int(v)
    return st


class AlphabetError(ValueError):
    """A stream's alphabet range(min-2, max+2) exceeds L = 1024 symbols: the
    reference's build_rans_table never terminates there (core/gpu_ans.py:73-84)."""


def encode_batch(x: torch.Tensor, bits, scale32: Optional[torch.Tensor] = None, deq_out: bool = False,
                 exact_size: bool = True, words_out: Optional[torch.Tensor] = None, wide="auto",
                 dither_seed=None, rht_signs: Optional[torch.Tensor] = None, escape: bool = True):
    """Compress a batch of chunks.

    x: (C, B, H, T, hd) fp16 / bf16 / fp32 CUDA tensor, hd % 8 == 0.
    bits: int or (C,) sequence of bits per dimension per chunk (3, 4, 5, ...).
    scale32: optional (C*B*H,) fp32 scales (otherwise from sigma^2 on the device).
    deq_out: also return q * scale32 in x's dtype (what update() hands to attention).
    exact_size: allocate the bitstream arena at its exact size (one host sync);
      else at a no-sync upper bound (10 bits per symbol).
    words_out: caller-provided arena (int32) large enough for the upper bound.
    wide: symbol staging width.  False: int8 (lattice symbols within int8; a
      chunk beyond sets LQ_ST_SYM_OVERFLOW in enc.status).  True: int16, for
      alphabets up to 1024 symbols.  "auto": int8 first, and if a chunk
      overflowed (one status read-back) the batch is redone on the wide path.
    escape: on the wide path, a coordinate whose alphabet exceeds 1024 symbols
      (where the reference's table normalisation never terminates) is coded
      as coarse symbols s >> k plus k raw low bits per vector (enc.escape; a
      format of this build, one host read of the shifts).  escape=False: such
      an alphabet raises AlphabetError when the status is read back
      (wide="auto" or True with exact_size) and is otherwise left in enc.status.
    dither_seed: int or (C,) ints: subtractive dither per chunk (the rotated
      path; the seeds are kept in enc.extra and decode_batch removes the dither).
    rht_signs: (C*B*H, hd) fp32 sign rows: the chunks are coded as their
      forward rotations w = RHT(x) (row of head h: sign row h), computed inside
      the scale and quantize kernels (hd a power of two <= 128); with deq_out,
      wide=True or an int8 overflow the rotation is materialised instead, with
      the same result.  deq is then the dequantised w.
    Returns (EncodedBatch, deq or None)."""
    lib = L.lib()
    x = _check_input(x)
    C, B, H, T, hd = x.shape
    if rht_signs is not None:
        rht_signs = _check_signs(rht_signs, C * B * H, hd, x.device)
        fused = not deq_out and wide is not True and hd <= 128
        if not fused:
            w = rotate_rows(x, rht_signs, inverse=False)
            return encode_batch(w, bits, scale32, deq_out, exact_size, words_out, wide, dither_seed,
                                escape=escape)
    dev = x.device
    nh, bph = B * H, T * hd // 8
    V = nh * bph
    nblk = (V + L.LQ_BLK - 1) // L.LQ_BLK
    dt = L.dtype_code(x.dtype)
    s = L.stream_ptr(dev)
    bits_t, scale32, scale16, sigma2, fastdiv = _head_scales(x, bits, scale32, rht_signs)
    # every block's 64 bytes of coset bits are written by the quantizer (bits of
    # vectors past the end are zero), so no fill
    coset_bits = _empty(C * nblk * L.LQ_BLK // 8, torch.uint8, dev)
    blk_n1 = _empty(C * nblk, torch.int32, dev)
    use_wide = wide is True
    esc = None
    # one zero fill: the status flags, the int8 path's histogram and a leading
    # zero before the chunks' word counts (so that one inclusive scan of
    # [0, w_0 .. w_{C-2}] gives the chunk bases)
    status, hist, cwz = _zero_views(dev, (C, torch.int32), (0 if use_wide else C * L.LQ_STREAMS * 256, torch.int32),
                                    (C + 1, torch.int64))
    deq = torch.empty_like(x) if deq_out else None
    tables = _empty(C * L.LQ_STREAMS * L.TABLE_BYTES, torch.uint8, dev)
    dseed = None
    if dither_seed is not None:
        ds = [int(dither_seed)] * C if isinstance(dither_seed, int) else [int(v) for v in dither_seed]
        if len(ds) != C:
            raise ValueError("dither_seed must be an int or one seed per chunk")
        dseed = torch.tensor(ds, dtype=torch.int64).to(dev)
    if not use_wide:
        sym = _empty(C * nblk * L.LQ_SYM_STRIDE, torch.int8, dev)
        if rht_signs is not None:
            L.check(lib.lq_chunk_quantize_rht(x.data_ptr(), dt, C, nh, bph, hd, rht_signs.data_ptr(),
                                              scale32.data_ptr(), sym.data_ptr(), coset_bits.data_ptr(),
                                              blk_n1.data_ptr(), hist.data_ptr(), status.data_ptr(), L.ptr(dseed), s),
                    "lq_chunk_quantize_rht")
        else:
            L.check(lib.lq_chunk_quantize(x.data_ptr(), dt, C, nh, bph, scale32.data_ptr(), fastdiv.data_ptr(),
                                          sym.data_ptr(), coset_bits.data_ptr(), blk_n1.data_ptr(), hist.data_ptr(),
                                          status.data_ptr(), L.ptr(deq), dt, L.ptr(dseed), s), "lq_chunk_quantize")
        if wide == "auto" and _status_or(status) & L.LQ_ST_SYM_OVERFLOW:
            if rht_signs is not None:   # the int16 path reads the materialised rotation
                w = rotate_rows(x, rht_signs, inverse=False)
                return encode_batch(w, bits, scale32, deq_out, exact_size, words_out, wide, dither_seed,
                                    escape=escape)
            use_wide = True
            status.zero_()
        else:
            L.check(lib.lq_chunk_tables(hist.data_ptr(), C, tables.data_ptr(), status.data_ptr(), s), "lq_chunk_tables")
    if use_wide:
        sym = _empty(C * nblk * L.LQ_SYM_STRIDE, torch.int16, dev)
        minmax = torch.empty(C * L.LQ_STREAMS, 2, dtype=torch.int32, device=dev)
        minmax[:, 0] = 2 ** 31 - 1
        minmax[:, 1] = -2 ** 31
        hist = _zeros(C * L.LQ_STREAMS * L.LQ_L, torch.int32, dev)
        L.check(lib.lq_chunk_quantize_wide(x.data_ptr(), dt, C, nh, bph, scale32.data_ptr(), fastdiv.data_ptr(),
                                           sym.data_ptr(), coset_bits.data_ptr(), blk_n1.data_ptr(), minmax.data_ptr(),
                                           status.data_ptr(), L.ptr(deq), dt, L.ptr(dseed), s),
                "lq_chunk_quantize_wide")
        if escape:
            esc, minmax = _plan_escape(minmax, C, nblk, V, sym, coset_bits, blk_n1, status, dev, s)
        L.check(lib.lq_chunk_hist_wide(sym.data_ptr(), blk_n1.data_ptr(), C, V, minmax.data_ptr(), hist.data_ptr(), s),
                "lq_chunk_hist_wide")
        L.check(lib.lq_chunk_tables_wide(hist.data_ptr(), minmax.data_ptr(), C, tables.data_ptr(), status.data_ptr(), s),
                "lq_chunk_tables_wide")
        if wide == "auto" or exact_size:
            st = _status_or(status)
            if st & L.LQ_ST_ALPHABET:
                raise AlphabetError("a stream's alphabet exceeds L = 1024 symbols (the reference's table "
                                    "normalisation never terminates there); use more bits or smaller chunks")
            if st & L.LQ_ST_SYM_OVERFLOW:
                raise AlphabetError("a lattice symbol does not fit int16")
    ws = lib.lq_chunk_encode_workspace(C, V)
    work = _empty(ws, torch.uint8, dev)
    ntask = C * L.LQ_STREAMS * nblk
    blk_off = _empty(ntask, torch.int32, dev)
    blk_state = _empty(ntask, torch.int16, dev)
    stream_nbits = _empty(C * L.LQ_STREAMS, torch.int64, dev)
    stream_state = _empty(C * L.LQ_STREAMS, torch.int32, dev)
    stream_woff = _empty(C * L.LQ_STREAMS, torch.int64, dev)
    chunk_words = cwz[1:]
    enc_fn = lib.lq_chunk_encode_wide if use_wide else lib.lq_chunk_encode
    L.check(enc_fn(sym.data_ptr(), blk_n1.data_ptr(), C, V, tables.data_ptr(), work.data_ptr(),
                   blk_off.data_ptr(), blk_state.data_ptr(), stream_nbits.data_ptr(),
                   stream_state.data_ptr(), stream_woff.data_ptr(), chunk_words.data_ptr(), s),
            "lq_chunk_encode_wide" if use_wide else "lq_chunk_encode")
    chunk_base = torch.cumsum(cwz[:C], 0)
    bound = words_bound(C, V)
    if words_out is not None:
        if words_out.numel() < bound:
            raise ValueError(f"words_out holds {words_out.numel()} words, needs {bound}")
        words = words_out
    elif exact_size:
        words = _empty(int(chunk_words.sum().item()) + 2, torch.int32, dev)   # decoder read-ahead slack
    else:
        words = _empty(bound, torch.int32, dev)
    L.check(lib.lq_chunk_pack(C, V, tables.data_ptr(), work.data_ptr(), blk_off.data_ptr(), stream_nbits.data_ptr(),
                              stream_woff.data_ptr(), chunk_base.data_ptr(), words.data_ptr(), s), "lq_chunk_pack")
    enc = EncodedBatch(n_chunks=C, n_heads=nh, bph=bph, shape=(B, H, T, hd), bits=bits_t, scale32=scale32,
                       scale16=scale16, sigma2=sigma2, coset_bits=coset_bits.view(C, -1), blk_n1=blk_n1.view(C, -1),
                       tables=tables, blk_off=blk_off, blk_state=blk_state, stream_nbits=stream_nbits,
                       stream_state=stream_state, stream_woff=stream_woff, chunk_words=chunk_words,
                       chunk_base=chunk_base, words=words, status=status, hist=hist,
                       extra={"wide": use_wide, "dither_seed": dseed, "esc": esc})
    return enc, deq


def decode_batch(enc: EncodedBatch, out_dtype: torch.dtype = torch.float16, out: Optional[torch.Tensor] = None,
                 lut_work: Optional[torch.Tensor] = None, rht_signs: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decompress every chunk of the batch: (C, B, H, T, hd) in out_dtype,
    fp16(q * float(scale16[head])) as _decompress_chunk computes it
    (llm/compressed_kv_cache.py:289-332).  rht_signs (C*B*H, hd): the rows are
    rotated back (inverse RHT of the fp32 dequantised rows, then out_dtype)
    inside the decoder for hd <= 128, else by a separate pass."""
    lib = L.lib()
    dev = enc.words.device
    C = enc.n_chunks
    if out is None:
        out = torch.empty((C,) + tuple(enc.shape), dtype=out_dtype, device=dev)
    if lut_work is None:
        lut_work = _empty(C * L.LQ_STREAMS * L.LQ_L, torch.int32, dev)
    # an escape plan still on its way to the host is not waited for: the
    # escaped decoder reads the shifts on the device (k_j = 0 decodes plainly)
    esc = enc.extra.get("esc")
    if esc is not None and esc.ready():
        esc = enc.escape
    if rht_signs is not None:
        hd = enc.shape[-1]
        rht_signs = _check_signs(rht_signs, C * enc.n_heads, hd, dev)
        if hd > 128:
            w = decode_batch(enc, out_dtype=torch.float32, lut_work=lut_work)
            out.copy_(rotate_rows(w, rht_signs, inverse=True, out_dtype=out.dtype))
            return out
    if esc is not None:   # chunks with coarse / fine coordinates
        hd = enc.shape[-1]
        L.check(lib.lq_chunk_decode_escaped(enc.words.data_ptr(), enc.chunk_base.data_ptr(), enc.stream_woff.data_ptr(),
                                            enc.blk_off.data_ptr(), enc.stream_nbits.data_ptr(),
                                            enc.blk_state.data_ptr(), enc.coset_bits.data_ptr(), enc.tables.data_ptr(),
                                            enc.scale16.data_ptr(), C, enc.n_heads, enc.bph,
                                            hd if rht_signs is not None else 0, L.ptr(rht_signs), esc.k.data_ptr(),
                                            esc.off.data_ptr(), esc.fine.data_ptr(), lut_work.data_ptr(),
                                            out.data_ptr(), L.dtype_code(out.dtype),
                                            L.ptr(enc.extra.get("dither_seed")), L.stream_ptr(dev)),
                "lq_chunk_decode_escaped")
        return out
    if rht_signs is not None:
        L.check(lib.lq_chunk_decode_rht(enc.words.data_ptr(), enc.chunk_base.data_ptr(), enc.stream_woff.data_ptr(),
                                        enc.blk_off.data_ptr(), enc.stream_nbits.data_ptr(), enc.blk_state.data_ptr(),
                                        enc.coset_bits.data_ptr(), enc.tables.data_ptr(), enc.scale16.data_ptr(), C,
                                        enc.n_heads, enc.bph, hd, rht_signs.data_ptr(), lut_work.data_ptr(),
                                        out.data_ptr(), L.dtype_code(out.dtype),
                                        L.ptr(enc.extra.get("dither_seed")), L.stream_ptr(dev)), "lq_chunk_decode_rht")
        return out
    L.check(lib.lq_chunk_decode(enc.words.data_ptr(), enc.chunk_base.data_ptr(), enc.stream_woff.data_ptr(),
                                enc.blk_off.data_ptr(), enc.stream_nbits.data_ptr(), enc.blk_state.data_ptr(),
                                enc.coset_bits.data_ptr(),
                                enc.blk_n1.data_ptr(), enc.tables.data_ptr(), enc.scale16.data_ptr(), C, enc.n_heads,
                                enc.bph, lut_work.data_ptr(), out.data_ptr(), L.dtype_code(out.dtype),
                                L.ptr(enc.extra.get("dither_seed")), L.stream_ptr(dev)), "lq_chunk_decode")
    return out


# ------------------------------------------------------------- host views --

def host_tables(enc: EncodedBatch):
    """(C*16) list of (lo, n_sym, n_symbols, status, freqs np.int32) read back from the device."""
    t = enc.tables.view(torch.int32).view(-1, L.TABLE_BYTES // 4).cpu().numpy()
    out = []
    for row in t:
        lo, n_sym, n_symbols, st = (int(v) for v in row[:4])
        enc_w = row[4:4 + n_sym].view(np.uint32)
        out.append((lo, n_sym, n_symbols, st, (enc_w & 0x7ff).astype(np.int32)))
    return out


def chunk_streams_host(enc: EncodedBatch, c: int):
    """Per present stream of chunk c: dict(coset, idx, n, lo, freqs, words, state, n_bits)."""
    tabs = host_tables(enc)
    nbits = enc.stream_nbits.cpu().numpy()
    state = enc.stream_state.cpu().numpy()
    woff = enc.stream_woff.cpu().numpy()
    base = int(enc.chunk_base[c].item())
    nw = int(enc.chunk_words[c].item())
    words = enc.words[base:base + nw].cpu().numpy().view(np.uint32)
    res = []
    for st in range(L.LQ_STREAMS):
        sid = c * L.LQ_STREAMS + st
        lo, n_sym, n_symbols, stt, freqs = tabs[sid]
        if n_sym == 0:
            continue
        w0 = int(woff[sid])
        nb = int(nbits[sid])
        res.append(dict(coset=st // 8, idx=st % 8, n=n_symbols, lo=lo, freqs=freqs,
                        words=words[w0:w0 + (nb + 31) // 32 + 1].copy(), state=int(state[sid]), n_bits=nb,
                        word_offset=w0, status=stt))
    return res


class PendingEncode:
    """Host-side completion of a batch that encode_batch_deferred wrote
    without any host sync.  A non-blocking copy of the chunks' status flags
    and word counts to pinned host memory is queued behind the encode, with an
    event.  result() (idempotent; waits for the event if needed) returns the
    final batch: the same batch with its bitstream arena trimmed to the exact
    size (a device copy; the bound-sized arena is released), or -- if a chunk's
    lattice symbols overflowed int8 -- the batch re-encoded on the int16 path
    from the kept input and the same scales.  Where encode_batch would raise
    AlphabetError, result() raises it, and again on every later call.
    ready() says, without blocking, whether result() can run without waiting."""

    # batches of at most this many vectors are not tracked: no copy or event is
    # queued per batch (those cost more than a small batch's encode on the
    # host); they are settled together by settle_many, or one by one on access
    TRACK_MIN_VECTORS = 1 << 16

    def __init__(self, enc: "EncodedBatch", x: torch.Tensor, bits, dither_seed):
        C = enc.n_chunks
        self._enc, self._x, self._bits, self._seed = enc, x, bits, dither_seed
        self._done = None
        self._error = None
        self._host = self._event = None
        self.tracked = C * enc.n_vectors > self.TRACK_MIN_VECTORS
        if self.tracked:
            self._host = torch.empty(2 * C, dtype=torch.int64, pin_memory=True)
            self._host.copy_(self._meta(), non_blocking=True)
            self._event = torch.cuda.Event()
            self._event.record(torch.cuda.current_stream(x.device))

    def _meta(self) -> torch.Tensor:
        return torch.cat([self._enc.status.to(torch.int64), self._enc.chunk_words])

    def retained_bytes(self) -> int:
        """Device bytes this unsettled batch keeps alive: the stacked input
        (kept for an int16 re-encode) and the bound-sized bitstream arena."""
        if self._done is not None or self._error is not None or self._enc is None:
            return 0
        return self._x.numel() * self._x.element_size() + self._enc.words.numel() * self._enc.words.element_size()

    def ready(self) -> bool:
        """Settled, or tracked and its read-back has arrived (non-blocking)."""
        if self._done is not None or self._error is not None:
            return True
        return self.tracked and self._event.query()

    def result(self) -> "EncodedBatch":
        if self._done is not None:
            return self._done
        if self._error is not None:
            raise self._error
        try:
            return self._settle()
        except AlphabetError as e:   # kept: every later access raises it again
            self._error = e
            self._enc = self._x = None
            raise

    def _settle(self, host=None) -> "EncodedBatch":
        if host is None:
            if self.tracked:
                self._event.synchronize()
                host = self._host
            else:
                host = self._meta().cpu()
        enc = self._enc
        C = enc.n_chunks
        st = 0
        for v in host[:C].tolist():
            st |= int(v)
        if st & L.LQ_ST_SYM_OVERFLOW:
            done, _ = encode_batch(self._x, self._bits, scale32=enc.scale32, exact_size=True, wide=True,
                                   dither_seed=self._seed)
            done.sigma2 = enc.sigma2   # the scales' sigma^2, as the first encode had them
        else:
            if st & L.LQ_ST_ALPHABET:
                raise AlphabetError("a stream's alphabet exceeds L = 1024 symbols (the reference's table "
                                    "normalisation never terminates there); use more bits or smaller chunks")
            n = int(host[C:].sum())
            enc.words = enc.words[:n + 2].clone()   # decoder read-ahead slack
            done = enc
        self._done = done
        self._enc = self._x = None
        return done


def settle_many(pends) -> None:
    """Settle pending batches with one device-to-host copy for all of them
    (their metadata concatenated on the device).  Batches whose alphabet check
    fails keep their AlphabetError for their next result()."""
    todo = [p for p in pends if p._done is None and p._error is None]
    if not todo:
        return
    host = torch.cat([p._meta() for p in todo]).cpu()
    o = 0
    for p in todo:
        n = 2 * p._enc.n_chunks
        try:
            p._done = p._settle(host[o:o + n])
            p._enc = p._x = None
        except AlphabetError as e:
            p._error = e
            p._enc = p._x = None
        o += n


def encode_batch_deferred(x: torch.Tensor, bits, deq_out: bool = False, dither_seed=None,
                          scale32: Optional[torch.Tensor] = None, sigma2: Optional[torch.Tensor] = None):
    """encode_batch with no host sync (int8 staging, bound-sized arena):
    returns (enc, deq, PendingEncode).  enc may be used for device work in
    stream order right away unless a chunk overflowed int8; the pending
    handle's result() is the batch to keep (see PendingEncode).  scale32 (and
    their sigma2): the chunks' scales when they were already computed
    (quantize_batch)."""
    x = _check_input(x)
    enc, deq = encode_batch(x, bits, scale32=scale32, deq_out=deq_out, exact_size=False, wide=False,
                            dither_seed=dither_seed)
    if scale32 is not None:
        enc.sigma2 = sigma2
    return enc, deq, PendingEncode(enc, x, bits, dither_seed)


# ------------------------------------------------------------ wire format --
#
# A self-describing, versioned byte form of an EncodedBatch for offload and
# restore (the reference has no serialisation of its chunks).  Layout, all
# little-endian:
#
#   b"LQE8RANS" | u32 version | u32 header bytes | header (UTF-8 JSON) |
#   payload (the fields in header order, each padded to 8 bytes) | u32 CRC-32
#
# The CRC covers every byte before it.  Per chunk the payload holds what
# decoding needs and nothing of the write path: the reference's merged
# bitstream words, coset bitmap and fp16 scales (its accounting,
# llm/compressed_kv_cache.py:113-119), then the compact tables (lo, n_sym,
# n_symbols, status + one uint16 frequency per symbol; cumulative
# frequencies and renormalisation shifts are rebuilt on load), the block
# checkpoints of present streams (uint32 bit offset + uint16 state), the
# per-block coset-1 counts (uint16) and the stream metadata.  Version 2 adds
# the coarse / fine escape (esc_k: 8 int32 shifts per chunk; fine: the raw
# low-bit words of every escaped coordinate in (chunk, coordinate) order);
# batches without escaped chunks are still written as version 1.

WIRE_MAGIC = b"LQE8RANS"
# the dither a seed stands for (lq_device.h dither8): 2 = 16-bit fields of two
# SplitMix64 outputs per vector; batches with a dither seed and no scheme 2
# were written with another dither and are refused
DITHER_SCHEME = 2
WIRE_VERSION = 2
WIRE_VERSIONS_READ = (1, 2)


class WireFormatError(ValueError):
    """A byte string that is not a valid serialised EncodedBatch."""


def _table_heads(enc: EncodedBatch) -> np.ndarray:
    t = enc.tables.view(torch.int32).view(-1, L.TABLE_BYTES // 4).cpu().numpy()
    return t


def to_bytes(enc: EncodedBatch) -> bytes:
    """Serialise an EncodedBatch (one device-to-host copy per field)."""
    import json
    import zlib
    C, S, nb = enc.n_chunks, L.LQ_STREAMS, enc.nblk
    t = _table_heads(enc)
    heads = np.ascontiguousarray(t[:, :4]).astype(np.int32)
    nsym = heads[:, 1].astype(np.int64)
    present = nsym > 0
    freqs = np.concatenate([(t[i, 4:4 + nsym[i]].view(np.uint32) & 0x7FF).astype(np.uint16) for i in range(C * S)]
                           or [np.zeros(0, np.uint16)])
    cw = enc.chunk_words.cpu().numpy().astype(np.int64)
    cb = enc.chunk_base.cpu().numpy().astype(np.int64)
    wall = enc.words.cpu().numpy().view(np.uint32)
    words = np.concatenate([wall[cb[c]:cb[c] + cw[c]] for c in range(C)] or [np.zeros(0, np.uint32)])
    off = enc.blk_off.cpu().numpy().view(np.uint32).reshape(C * S, nb)[present]
    st = enc.blk_state.cpu().numpy().view(np.uint16).reshape(C * S, nb)[present]
    fields = [
        ("bits", enc.bits.cpu().numpy().astype(np.int32)),
        ("status", enc.status.cpu().numpy().astype(np.int32)),
        ("scale32", enc.scale32.cpu().numpy().astype(np.float32)),
        ("scale16", enc.scale16.cpu().numpy().astype(np.float16)),
        ("chunk_words", cw),
        ("words", words),
        ("stream_nbits", enc.stream_nbits.cpu().numpy().astype(np.int64)),
        ("stream_state", enc.stream_state.cpu().numpy().astype(np.int32)),
        ("stream_woff", enc.stream_woff.cpu().numpy().astype(np.int64)),
        ("table_heads", heads.reshape(-1)),
        ("table_freqs", freqs),
        ("coset_bits", enc.coset_bits.cpu().numpy().astype(np.uint8).reshape(-1)),
        ("blk_n1", enc.blk_n1.cpu().numpy().astype(np.uint16).reshape(-1)),
        ("blk_off", off.reshape(-1)),
        ("blk_state", st.reshape(-1)),
    ]
    if enc.sigma2 is not None:
        fields.append(("sigma2", enc.sigma2.cpu().numpy().astype(np.float32)))
    extra = {}
    ds = enc.extra.get("dither_seed")
    if ds is not None:
        fields.append(("dither_seed", ds.cpu().numpy().astype(np.int64)))
        extra["dither_scheme"] = DITHER_SCHEME
    if "rht" in enc.extra:
        layers, kvs = enc.extra["rht"]
        extra["rht"] = [[int(v) for v in layers], [int(v) for v in kvs]]
    esc = enc.escape
    if esc is not None:
        kh = esc.k_host.astype(np.int32).reshape(-1)
        offs = esc.off.cpu().numpy()
        fall = esc.fine.cpu().numpy().view(np.uint32)
        fine = [fall[o:o + 16 * nb * int(k)] for o, k in zip(offs, kh) if k]
        fields.append(("esc_k", kh))
        fields.append(("fine", np.concatenate(fine) if fine else np.zeros(0, np.uint32)))
    header = {"n_chunks": C, "n_heads": enc.n_heads, "bph": enc.bph, "shape": [int(v) for v in enc.shape],
              "fields": [[n, a.dtype.str, int(a.size)] for n, a in fields], "extra": extra}
    hb = json.dumps(header, separators=(",", ":")).encode()
    version = WIRE_VERSION if esc is not None else 1
    parts = [WIRE_MAGIC, np.uint32(version).tobytes(), np.uint32(len(hb)).tobytes(), hb]
    pos = sum(len(p) for p in parts)
    for _, a in fields:
        pad = (-pos) % 8
        parts.append(b"\0" * pad)
        b = np.ascontiguousarray(a).tobytes()
        parts.append(b)
        pos += pad + len(b)
    body = b"".join(parts)
    return body + np.uint32(zlib.crc32(body) & 0xFFFFFFFF).tobytes()


def _check_wire_geometry(C, nh, bph, shape, arrs):
    """Field sizes against the batch geometry (the decoder indexes by them)."""
    S, B = L.LQ_STREAMS, L.LQ_BLK
    if C < 1 or nh < 1 or bph < 1 or bph > (1 << 30) or len(shape) != 4:
        raise WireFormatError("bad batch geometry")
    if shape[0] * shape[1] != nh or shape[2] * shape[3] != 8 * bph:
        raise WireFormatError("chunk shape does not match n_heads x bph")
    nb = (nh * bph + B - 1) // B
    need = {"bits": C, "status": C, "scale32": C * nh, "scale16": C * nh, "chunk_words": C,
            "stream_nbits": C * S, "stream_state": C * S, "stream_woff": C * S, "table_heads": C * S * 4,
            "coset_bits": C * nb * B // 8, "blk_n1": C * nb, "words": None, "table_freqs": None,
            "blk_off": None, "blk_state": None}
    for name, n in need.items():
        if name not in arrs:
            raise WireFormatError(f"missing field {name}")
        if n is not None and arrs[name].size != n:
            raise WireFormatError(f"field {name} holds {arrs[name].size} values, the geometry needs {n}")
    for name, n in (("sigma2", C * nh), ("dither_seed", C), ("esc_k", C * 8)):
        if name in arrs and arrs[name].size != n:
            raise WireFormatError(f"field {name} holds {arrs[name].size} values, the geometry needs {n}")


def _check_wire_streams(C, nv, nb, present, arrs, off, st):
    """Cross-checks of every value the chunk decoder uses as an address or a
    count: the reference word layout of the merged bitstream (present streams
    in stream order, ceil(n_bits / 32) + 1 words each, the total in
    chunk_words), block checkpoints (bit offsets from 0, non-decreasing, at
    most the stream's n_bits; states in [L, 2L)), per-block coset-1 counts equal
    to the coset bitmap's, and a coset's streams present exactly when it holds
    vectors."""
    S, B = L.LQ_STREAMS, L.LQ_BLK
    nbits = arrs["stream_nbits"].astype(np.int64).reshape(C, S)
    woff = arrs["stream_woff"].astype(np.int64).reshape(C, S)
    cw = arrs["chunk_words"].astype(np.int64)
    if np.any(nbits < 0) or np.any(nbits[~present] != 0) or np.any(nbits >= (1 << 32)):
        raise WireFormatError("stream bit counts out of range")
    per = np.where(present, (nbits + 31) // 32 + 1, 0)
    if not np.array_equal(woff, np.cumsum(per, 1) - per) or not np.array_equal(cw, per.sum(1)):
        raise WireFormatError("stream word offsets do not follow the merged bitstream layout")
    o = off.reshape(C, S, nb).astype(np.int64)
    p = present
    if np.any(o[p][:, 0] != 0) or np.any(np.diff(o[p], axis=1) < 0) or np.any(o[p] > nbits[p][:, None]):
        raise WireFormatError("block checkpoint offsets out of order or past the stream end")
    sv = st.reshape(C, S, nb).astype(np.int64)
    if np.any(sv[p] < L.LQ_L) or np.any(sv[p] >= 2 * L.LQ_L):
        raise WireFormatError("block checkpoint states outside [L, 2L)")
    bits = np.unpackbits(arrs["coset_bits"].reshape(C, nb, B // 8), axis=2, bitorder="little")
    valid = np.minimum(B, nv - np.arange(nb) * B)
    bits[:, np.arange(B)[None, :] >= valid[:, None]] = 0
    n1 = bits.sum(2)
    if not np.array_equal(n1, arrs["blk_n1"].astype(np.int64).reshape(C, nb)):
        raise WireFormatError("per-block coset-1 counts disagree with the coset bitmap")
    tot1 = n1.sum(1)
    if (np.any(present[:, 8:] != (tot1 > 0)[:, None]) or
            np.any(present[:, :8] != (nv - tot1 > 0)[:, None])):
        raise WireFormatError("stream presence disagrees with the coset counts")


def from_bytes(buf, device=None) -> EncodedBatch:
    """Restore an EncodedBatch on `device` (default: the current CUDA device).
    Raises WireFormatError on a bad magic, version, checksum or layout."""
    import json
    import zlib
    mv = memoryview(buf)
    if len(mv) < 20 or bytes(mv[:8]) != WIRE_MAGIC:
        raise WireFormatError("not an LQE8RANS chunk batch")
    version = int(np.frombuffer(mv[8:12], np.uint32)[0])
    if version not in WIRE_VERSIONS_READ:
        raise WireFormatError(f"unsupported wire format version {version} (this build reads "
                              f"{', '.join(str(v) for v in WIRE_VERSIONS_READ)})")
    crc = int(np.frombuffer(mv[len(mv) - 4:], np.uint32)[0])
    if zlib.crc32(mv[:len(mv) - 4]) & 0xFFFFFFFF != crc:
        raise WireFormatError("checksum mismatch: the chunk batch is corrupted")
    hl = int(np.frombuffer(mv[12:16], np.uint32)[0])
    try:
        header = json.loads(bytes(mv[16:16 + hl]).decode())
        C, nh, bph = int(header["n_chunks"]), int(header["n_heads"]), int(header["bph"])
        shape = tuple(int(v) for v in header["shape"])
    except (ValueError, KeyError, TypeError) as e:
        raise WireFormatError(f"bad header: {e}") from None
    pos = 16 + hl
    end = len(mv) - 4
    arrs = {}
    if not isinstance(header.get("fields"), list):
        raise WireFormatError("bad header: no field list")
    for name, dts, n in header["fields"]:
        pos += (-pos) % 8
        dt = np.dtype(dts)
        nbytes = dt.itemsize * int(n)
        if pos + nbytes > end:
            raise WireFormatError(f"truncated field {name}")
        arrs[name] = np.frombuffer(mv[pos:pos + nbytes], dt).copy()
        pos += nbytes
    S = L.LQ_STREAMS
    _check_wire_geometry(C, nh, bph, shape, arrs)
    nv = nh * bph
    nb = (nv + L.LQ_BLK - 1) // L.LQ_BLK
    heads = arrs["table_heads"].reshape(C * S, 4)
    nsym = heads[:, 1].astype(np.int64)
    if arrs["table_freqs"].size != int(nsym.sum()) or np.any(nsym < 0) or np.any(nsym > L.LQ_MAXSYM):
        raise WireFormatError("inconsistent tables")
    # rebuild the device tables: enc[j] = f | cum << 11 | (11 - bitlen(f)) << 21
    tab = np.zeros((C * S, L.TABLE_BYTES // 4), np.uint32)
    tab[:, :4] = heads.view(np.uint32)
    f_all = arrs["table_freqs"].astype(np.uint32)
    o = 0
    for i in range(C * S):
        k = int(nsym[i])
        if k:
            f = f_all[o:o + k]
            if np.any(f == 0) or int(f.sum()) != L.LQ_L:
                raise WireFormatError("table frequencies do not sum to L")
            cum = np.cumsum(f) - f
            bl = np.frexp(f.astype(np.float64))[1].astype(np.uint32)   # bit length of f
            tab[i, 4:4 + k] = f | (cum.astype(np.uint32) << 11) | ((11 - bl) << 21)
        o += k
    present = nsym > 0
    npres = int(present.sum())
    off = np.zeros((C * S, nb), np.uint32)
    st = np.full((C * S, nb), L.LQ_L, np.uint16)
    if arrs["blk_off"].size != npres * nb or arrs["blk_state"].size != npres * nb:
        raise WireFormatError("inconsistent checkpoints")
    off[present] = arrs["blk_off"].reshape(npres, nb)
    st[present] = arrs["blk_state"].reshape(npres, nb)
    cw = arrs["chunk_words"].astype(np.int64)
    if arrs["words"].size != int(cw.sum()):
        raise WireFormatError("inconsistent bitstream length")
    _check_wire_streams(C, nv, nb, present.reshape(C, S), arrs, off, st)
    if ("esc_k" in arrs) != ("fine" in arrs) or ("esc_k" in arrs and version < 2):
        raise WireFormatError("inconsistent escape fields")
    if "esc_k" in arrs:
        kh = arrs["esc_k"].astype(np.int64)
        if np.any(kh < 0) or np.any(kh > 7) or arrs["fine"].size != int(16 * nb * kh.sum()):
            raise WireFormatError("escape shifts out of range or low-bit words of the wrong length")
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())

    def T(a, dt):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dt).to(dev)

    words = np.concatenate([arrs["words"], np.zeros(2, np.uint32)])   # decoder read-ahead slack
    enc = EncodedBatch(
        n_chunks=C, n_heads=nh, bph=bph, shape=shape, bits=T(arrs["bits"], torch.int32),
        scale32=T(arrs["scale32"], torch.float32), scale16=T(arrs["scale16"], torch.float16),
        sigma2=T(arrs["sigma2"], torch.float32) if "sigma2" in arrs else None,
        coset_bits=T(arrs["coset_bits"].reshape(C, -1), torch.uint8),
        blk_n1=T(arrs["blk_n1"].astype(np.int32).reshape(C, nb), torch.int32),
        tables=torch.from_numpy(tab.view(np.uint8).reshape(-1).copy()).to(dev),
        blk_off=torch.from_numpy(off.view(np.int32).reshape(-1).copy()).to(dev),
        blk_state=torch.from_numpy(st.view(np.int16).reshape(-1).copy()).to(dev),
        stream_nbits=T(arrs["stream_nbits"], torch.int64), stream_state=T(arrs["stream_state"], torch.int32),
        stream_woff=T(arrs["stream_woff"], torch.int64), chunk_words=T(cw, torch.int64),
        chunk_base=T(np.cumsum(cw) - cw, torch.int64),
        words=torch.from_numpy(words.view(np.int32).copy()).to(dev), status=T(arrs["status"], torch.int32))
    if "dither_seed" in arrs:
        if header.get("extra", {}).get("dither_scheme") != DITHER_SCHEME:
            raise WireFormatError("the batch's dither seeds stand for another dither scheme")
        enc.extra["dither_seed"] = T(arrs["dither_seed"], torch.int64)
    if "rht" in header.get("extra", {}):
        layers, kvs = header["extra"]["rht"]
        enc.extra["rht"] = (list(layers), list(kvs))
    if "esc_k" in arrs and arrs["esc_k"].any():
        kh = arrs["esc_k"].astype(np.int32).reshape(C, 8)
        per = 16 * nb * kh.astype(np.int64).reshape(-1)
        offs = np.cumsum(per) - per
        fine = np.concatenate([arrs["fine"].astype(np.uint32), np.zeros(1, np.uint32)])
        enc.extra["esc"] = Escape(k=T(kh, torch.int32), off=T(offs, torch.int64),
                                  fine=torch.from_numpy(fine.view(np.int32).copy()).to(dev), k_host=kh)
    return enc


def save_batch(path, enc: EncodedBatch) -> int:
    """Write an EncodedBatch to `path`; returns the bytes written."""
    b = to_bytes(enc)
    with open(path, "wb") as f:
        f.write(b)
    return len(b)


def load_batch(path, device=None) -> EncodedBatch:
    """Read an EncodedBatch written by save_batch."""
    with open(path, "rb") as f:
        return from_bytes(f.read(), device)
