"""Decode-step attention straight from the compressed KV prefix.

out = softmax(q K^T / sqrt(128)) V over a prefix held as E8 + rANS chunks
(the reference's bitstreams, llm/compressed_kv_cache.py:176-287) followed by
an fp16 residual tail.  K and V are dequantised the way _decompress_chunk
does (lattice point times the fp16-stored scale,
llm/compressed_kv_cache.py:289-332).  The scores are computed straight from
K's bitstreams (K is never materialised); V is decoded to fp16 in workspace
by the chunk decoder and consumed by a split-token softmax . V pass, whose
records are merged with the tail's by log-sum-exp (lq_decode_attention).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from .. import _lib as L
from ..codec import EncodedBatch


def chunk_batch(enc: EncodedBatch) -> L.ChunkBatch:
    """lq_chunk_batch view of an EncodedBatch (device pointers, no copies)."""
    return L.ChunkBatch(words=enc.words.data_ptr(), chunk_base=enc.chunk_base.data_ptr(),
                        stream_woff=enc.stream_woff.data_ptr(), blk_off=enc.blk_off.data_ptr(),
                        stream_nbits=enc.stream_nbits.data_ptr(), blk_state=enc.blk_state.data_ptr(), coset_bits=enc.coset_bits.data_ptr(),
                        blk_n1=enc.blk_n1.data_ptr(), tables=enc.tables.data_ptr(), scale16=enc.scale16.data_ptr(),
                        n_chunks=enc.n_chunks, n_heads=enc.n_heads, bph=enc.bph)


def attn_workspace(enc: EncodedBatch, group: int, device=None) -> torch.Tensor:
    n = L.lib().lq_attn_workspace(enc.n_chunks, enc.n_heads, enc.bph, group)
    if n < 0:
        raise ValueError("bad attention geometry")
    return torch.empty(int(n), dtype=torch.uint8, device=device or enc.words.device)


def decode_attention(k: EncodedBatch, v: EncodedBatch, q: torch.Tensor, tail_k: Optional[torch.Tensor] = None,
                     tail_v: Optional[torch.Tensor] = None, work: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """q: (B, Hq, 1, 128) fp16 (one new token); k / v: chunk batches of
    (B, Hkv, T, 128) chunks, T % 32 == 0; tail_k / tail_v: (B, Hkv, Tt, 128)
    fp16, Tt <= 1024, or None.  Returns (B, Hq, 1, 128) fp16."""
    lib = L.lib()
    if k.shape != v.shape or k.n_chunks != v.n_chunks:
        raise ValueError("K and V batches must have the same geometry")
    if k.escape is not None or v.escape is not None:
        raise ValueError("decode attention reads the reference's chunk format; escaped chunks (alphabets beyond "
                         "L = 1024) are decoded with codec.decode_batch")
    B, Hkv, T, hd = k.shape
    if hd != 128 or T % 32:
        raise ValueError("decode attention needs head_dim 128 and a multiple of 32 tokens per chunk")
    if q.dtype != torch.float16 or q.dim() != 4 or q.shape[0] != B or q.shape[2] != 1 or q.shape[3] != hd:
        raise ValueError("q must be (B, Hq, 1, 128) fp16")
    Hq = q.shape[1]
    if Hq % Hkv or Hq // Hkv not in (1, 2, 4, 8):
        raise ValueError("query heads must be 1, 2, 4 or 8 times the kv heads")
    group = Hq // Hkv
    dev = k.words.device
    qc = q.to(dev).contiguous()
    tt = 0
    pk = pv = None
    if tail_k is not None and tail_k.shape[2] > 0:
        if tail_k.shape != tail_v.shape or tail_k.shape[:2] != (B, Hkv) or tail_k.shape[3] != hd:
            raise ValueError("tail K / V must be (B, Hkv, Tt, 128)")
        tt = int(tail_k.shape[2])
        if tt > 1024:
            raise ValueError("tail longer than 1024 tokens: compress it into the prefix first")
        pk = tail_k.to(device=dev, dtype=torch.float16).contiguous()
        pv = tail_v.to(device=dev, dtype=torch.float16).contiguous()
    if work is None:
        work = attn_workspace(k, group, dev)
    elif work.numel() < lib.lq_attn_workspace(k.n_chunks, k.n_heads, k.bph, group):
        raise ValueError("attention workspace too small")
    if out is None:
        out = torch.empty(B, Hq, 1, hd, dtype=torch.float16, device=dev)
    kb, vb = chunk_batch(k), chunk_batch(v)
    with torch.cuda.device(dev):
        L.check(lib.lq_decode_attention(ctypes.addressof(kb), ctypes.addressof(vb), qc.data_ptr(), group, L.ptr(pk),
                                        L.ptr(pv), tt, work.data_ptr(), out.data_ptr(), L.stream_ptr(dev)),
                "lq_decode_attention")
    return out
