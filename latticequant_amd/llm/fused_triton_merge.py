"""Single-pass merge of fixed-rate packed vectors with fp16 fallback vectors
(API of reference llm/fused_triton_merge.py).

Name kept for import compatibility; the kernel is hand-written HIP
(lq_fused_merge).  Block i of the chunk is unpacked from
packed[rank_repr(i)] when repr_mask[i] is set, else copied from
fallback[rank_fb(i)]; the ranks are prefix counts of the mask computed in the
kernel (tile counts, one scan, wave ballots) instead of two torch.cumsum
passes (llm/fused_triton_merge.py:150-152).  head = i // blocks_per_head.

c7's low bit follows unpack_e8's floor-mod parity (core/compact_storage.py:203-208).
The reference kernel computes psum % 2 on signed values (llm/fused_triton_merge.py:86),
which Triton lowers to a truncating remainder, so its c7 is off by -2 whenever the
partial sum is negative and odd; that defect is not reproduced.
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .. import codec
from .compressed_kv_cache import CompressedChunk, CompressedKVCache, OptimizedChunk


def fused_decompress_chunk(chunk: CompressedChunk) -> torch.Tensor:
    """Fixed-rate chunk -> fp16 (B, H, T, hd).  llm/fused_triton_merge.py:137-172"""
    dev = chunk.repr_mask.device
    if dev.type != "cuda":
        raise ValueError("chunk tensors must live on a ROCm device")
    batch, heads, seq, hd = chunk.orig_shape
    bph = chunk.blocks_per_head
    total = batch * heads * bph
    assert total * 8 == batch * heads * seq * hd
    bits = chunk.bits_per_dim
    rm = chunk.repr_mask
    mask = rm.view(torch.uint8) if rm.dtype == torch.bool and rm.is_contiguous() else rm.to(torch.uint8).contiguous()
    if mask.numel() != total:
        raise ValueError("repr_mask must hold one flag per block")
    packed = chunk.packed.contiguous()
    fallback = chunk.fallback.to(torch.float16).contiguous()
    n_repr = int(packed.shape[0])
    if packed.dim() != 2 or (n_repr and packed.shape[1] != bits):
        raise ValueError(f"packed must be (n_repr, {bits}) uint8")
    # the kernel indexes packed / fallback by mask ranks and clamps ranks past
    # their row counts; LQ_DEBUG_CHECKS=1 also checks the counts on the host (a sync)
    if L.debug_checks():
        n_set = int(mask.sum().item())
        if n_set != n_repr or total - n_set != fallback.shape[0]:
            raise ValueError(f"mask selects {n_set} packed / {total - n_set} fallback blocks, chunk holds "
                             f"{n_repr} / {fallback.shape[0]}")
    sc = chunk.scales.to(device=dev, dtype=torch.float32).contiguous()
    if sc.numel() < batch * heads:
        raise ValueError("one scale per head required")
    out = torch.empty(total * 8, dtype=torch.float16, device=dev)
    toff = chunk.tile_offsets
    if toff is not None:   # tile offsets from the encoder: no look-back pass
        if toff.dtype != torch.int64 or toff.numel() != (total + 1023) // 1024 or toff.device != dev:
            raise ValueError("tile_offsets must hold one int64 per 1024-vector tile on the chunk's device")
        with torch.cuda.device(dev):
            L.check(L.lib().lq_compact_merge(packed.data_ptr(), n_repr, bits, fallback.data_ptr(),
                                             int(fallback.shape[0]), mask.data_ptr(), sc.data_ptr(), total, bph,
                                             toff.contiguous().data_ptr(), out.data_ptr(), L.stream_ptr(dev)),
                    "lq_compact_merge")
        return out.reshape(batch, heads, seq, hd)
    work = torch.empty(max(int(L.lib().lq_merge_workspace(total)), 8), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        L.check(L.lib().lq_fused_merge(packed.data_ptr(), n_repr, bits, fallback.data_ptr(), int(fallback.shape[0]),
                                       mask.data_ptr(), sc.data_ptr(), total, bph, work.data_ptr(), out.data_ptr(),
                                       L.stream_ptr(dev)),
                "lq_fused_merge")
    if L.debug_checks():   # the look-back error word after the tile words (a sync)
        tiles = (total + 1023) // 1024
        if int(work[(tiles + 1) * 8:(tiles + 1) * 8 + 4].view(torch.int32).item()):
            raise codec.LookbackError("lq_fused_merge: a tile look-back wait did not end; the output is invalid")
    return out.reshape(batch, heads, seq, hd)


class FusedTritonKVCache(CompressedKVCache):
    """CompressedKVCache whose _decompress_chunk also accepts fixed-rate chunks
    (llm/fused_triton_merge.py:181-185)."""

    def _decompress_chunk(self, chunk) -> torch.Tensor:
        if isinstance(chunk, OptimizedChunk):
            return super()._decompress_chunk(chunk)
        return fused_decompress_chunk(chunk)
