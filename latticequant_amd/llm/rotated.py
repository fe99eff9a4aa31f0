"""Rotated and dithered compressed KV: the long-context batched write/read path.

Per 128-dim vector: the HeadRHT rotation of its (layer, head, K/V)
(seed layer*10000 + head*10 + kv, llm/perplexity_eval.py:35-61; transform
core/pipeline.py:49-118), then a subtractive dither, then the chunk codec
(E8 nearest point at b bits per dimension, per-stream rANS; the reference's
bitstream format).  Reading inverts it: decode, subtract the dither, scale by
the fp16-stored scale, inverse rotation.

The dither is build-defined (the reference dithers only its scalar
quantizers, ddt/dithered_comparison.py:117-147): vector v of a chunk gets
d in [-1, 1)^8 from SplitMix64 of (seed, v), a fundamental domain of
2Z^8 ⊂ E8, so the reconstruction error (Q(x/a + d) - d) a - x is uniform on
a times the E8 Voronoi cell and independent of x (per-dimension MSE
G(E8) a^2, G(E8) = 0.0716821).  Chunk seeds default to the HeadRHT-style
layer*10000 + kv*10 + 7.

Everything runs in the library's kernels: lq_head_scales_rht and
lq_chunk_quantize_rht rotate each row in registers (no rotated copy in
memory) before the scale sums and the nearest-point search, then tables,
encode, pack; lq_chunk_decode_rht removes the dither and rotates each row back
before its fp16 store.  The rotation's fp32 arithmetic is the one lq_rht
applies to a materialised copy, so the streams are the same either way.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

from .. import codec
from ..core.pipeline import _rht, sign_vector

__all__ = ["chunk_signs", "default_dither_seed", "encode_rotated", "decode_rotated", "G_E8"]

G_E8 = 0.0716821   # normalised second moment of E8 (Conway & Sloane, SPLAG ch. 21)

_SIGN_CACHE = {}


def _signs(head_dim: int, layer: int, head: int, kv: int) -> torch.Tensor:
    key = (head_dim, layer, head, kv)
    if key not in _SIGN_CACHE:
        _SIGN_CACHE[key] = sign_vector(head_dim, layer * 10000 + head * 10 + kv)
    return _SIGN_CACHE[key]


def chunk_signs(shape, layers: Sequence[int], kvs: Sequence[int]) -> torch.Tensor:
    """Sign rows of a (C, B, H, T, hd) batch: row (c * B + b) * H + h is the
    HeadRHT signs of (layers[c], h, kvs[c]) (CPU fp32)."""
    C, B, H, _, hd = shape
    rows = []
    for c in range(C):
        per = [_signs(hd, layers[c], h, kvs[c]) for h in range(H)]
        rows.extend(per * B)
    return torch.stack(rows)


_DEV_SIGNS = {}


def _device_signs(shape, layers, kvs, device) -> torch.Tensor:
    """chunk_signs on the device, kept per (geometry, layers, K/V, device): the
    sustained write / read loops then issue no host-to-device copy per call.
    Kernels on any stream may read a cached entry: its copy is complete before
    it is first returned, and entries are never freed while the process runs;
    past 256 entries a new key gets a per-call copy, read on the current
    stream only."""
    C, B, H, _, hd = shape
    key = (C, B, H, hd, tuple(layers), tuple(kvs), str(device))
    t = _DEV_SIGNS.get(key)
    if t is None:
        t = chunk_signs(shape, layers, kvs).to(device)
        if len(_DEV_SIGNS) < 256:
            if t.is_cuda:
                torch.cuda.current_stream(t.device).synchronize()
            _DEV_SIGNS[key] = t
    return t


def prepare_signs(shape, layers, kvs, device) -> torch.Tensor:
    """Draw and upload the sign rows of a chunk geometry once (the reference
    builds its HeadRHT signs when the object is made,
    llm/perplexity_eval.py:35-61); later encode_rotated / decode_rotated calls
    with the same (geometry, layers, K/V) find them on the device."""
    C = shape[0]
    layers, kvs = _lists(C, layers, kvs)
    return _device_signs(shape, layers, kvs, device)


def default_dither_seed(layer: int, kv: int) -> int:
    return layer * 10000 + kv * 10 + 7


def _lists(C, layers, kvs):
    layers = [int(v) for v in (layers if isinstance(layers, (list, tuple)) else [layers] * C)]
    kvs = [int(v) for v in (kvs if isinstance(kvs, (list, tuple)) else [kvs] * C)]
    if len(layers) != C or len(kvs) != C:
        raise ValueError("layers / kvs: one value per chunk")
    return layers, kvs


def encode_rotated(x: torch.Tensor, bits, layers, kvs, dither_seeds: Optional[Sequence[int]] = None,
                   deq_out: bool = False, **kw) -> Tuple[codec.EncodedBatch, Optional[torch.Tensor]]:
    """Rotate, dither and compress a (C, B, H, T, hd) batch (chunk c belongs to
    layer layers[c], K (0) or V (1) kvs[c]).  The rotation runs inside the
    scale and quantize kernels (no rotated copy in memory) unless deq_out asks
    for the reconstruction.  Returns (EncodedBatch, deq or None), deq being the
    reconstruction in x's dtype (what a cache would hand to attention)."""
    if x.dim() != 5:
        raise ValueError("x must be (C, B, H, T, hd)")
    C, B, H, T, hd = x.shape
    layers, kvs = _lists(C, layers, kvs)
    seeds = list(dither_seeds) if dither_seeds is not None else [default_dither_seed(l, k) for l, k in zip(layers, kvs)]
    signs = _device_signs(x.shape, layers, kvs, x.device)
    enc, deq = codec.encode_batch(x, bits, deq_out=deq_out, dither_seed=seeds, rht_signs=signs, **kw)
    enc.extra["rht"] = (layers, kvs)
    if deq is not None:
        deq = _rht(deq, signs, inverse=True, rows_per_sign=T, out_dtype=x.dtype)
    return enc, deq


def decode_rotated(enc: codec.EncodedBatch, out_dtype: torch.dtype = torch.float16,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode a batch written by encode_rotated: (C, B, H, T, hd) in out_dtype
    (out's dtype when out is given); the inverse rotation runs inside the
    decoder."""
    layers, kvs = enc.extra["rht"]
    C = enc.n_chunks
    B, H, T, hd = enc.shape
    signs = _device_signs((C, B, H, T, hd), layers, kvs, enc.words.device)
    return codec.decode_batch(enc, out_dtype=out.dtype if out is not None else out_dtype, out=out, rht_signs=signs)
