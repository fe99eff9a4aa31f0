"""Unfused fixed-rate chunk decompression (API of reference
llm/triton_kv_integration.py): fallback vectors are scattered to the
out-of-range positions, the packed vectors go through the 4-bit (or b-bit)
unpack kernel and are scattered to the rest.  Same result as
fused_decompress_chunk; kept for callers of the reference's module.
"""
from __future__ import annotations

import torch

from ..core.triton_dequant import unpack_e8_dequant
from .compressed_kv_cache import CompressedChunk, CompressedKVCache, OptimizedChunk


def triton_decompress_chunk(chunk: CompressedChunk) -> torch.Tensor:
    """llm/triton_kv_integration.py:34-81"""
    dev = chunk.repr_mask.device
    batch, heads, seq, hd = chunk.orig_shape
    bph = chunk.blocks_per_head
    total = batch * heads * bph
    assert total * 8 == batch * heads * seq * hd, \
        f"Block count mismatch: {total}*8 != {batch}*{heads}*{seq}*{hd}"
    mask = chunk.repr_mask.to(device=dev, dtype=torch.bool)
    result = torch.empty(total, 8, dtype=torch.float16, device=dev)
    if chunk.fallback.shape[0] > 0:
        result[~mask] = chunk.fallback.to(torch.float16)
    if chunk.packed.shape[0] > 0:
        result[mask] = unpack_e8_dequant(chunk.packed, chunk.scales, chunk.repr_head_ids, chunk.bits_per_dim)
    return result.reshape(batch, heads, seq, hd)


class TritonCompressedKVCache(CompressedKVCache):
    """llm/triton_kv_integration.py:88-94"""

    def _decompress_chunk(self, chunk) -> torch.Tensor:
        if isinstance(chunk, OptimizedChunk):
            return super()._decompress_chunk(chunk)
        return triton_decompress_chunk(chunk)
