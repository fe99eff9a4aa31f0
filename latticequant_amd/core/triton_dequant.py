"""4-bit fixed-rate E8 unpack + dequant (API of reference core/triton_dequant.py).

The module keeps the reference's name for import compatibility; the kernel is
hand-written HIP (lq_unpack_compact), not Triton.  Per vector: one 4-byte
big-endian word -> coset, c0..c6 (4-bit, bias -8), c7 = 2 * upper +
parity(c0 + .. + c6) - 8; out = fp16((c + 0.5 * coset) * scales[head_idx]).
The parity is the floor-mod one of unpack_e8 (the reference kernel's
abs(psum) % 2 at core/triton_dequant.py:104 gives the same bit).
"""
from __future__ import annotations

import torch

from .. import _lib as L


def triton_unpack_e8_4bit(packed: torch.Tensor, scales: torch.Tensor, head_indices: torch.Tensor) -> torch.Tensor:
    """(N, 4) uint8, (H,) fp32 scales, (N,) int32 head index -> (N, 8) fp16.
    core/triton_dequant.py:139-177"""
    assert packed.dtype == torch.uint8
    assert packed.shape[1] == 4
    assert packed.is_cuda
    return unpack_e8_dequant(packed, scales, head_indices, 4)


def unpack_e8_dequant(packed: torch.Tensor, scales: torch.Tensor, head_indices: torch.Tensor,
                      bits_per_dim: int) -> torch.Tensor:
    """b-bit (b in 3, 4, 5) generalisation of triton_unpack_e8_4bit."""
    if not packed.is_cuda:
        raise ValueError("packed must be a ROCm device tensor")
    if packed.dtype != torch.uint8 or packed.dim() != 2 or packed.shape[1] != bits_per_dim:
        raise ValueError(f"packed must be (N, {bits_per_dim}) uint8")
    dev = packed.device
    n = packed.shape[0]
    p = packed.contiguous()
    sc = scales.to(device=dev, dtype=torch.float32).contiguous()
    hi = head_indices.to(device=dev, dtype=torch.int32).contiguous()
    if hi.numel() != n:
        raise ValueError("head_indices must hold one index per vector")
    if sc.numel() == 0:
        raise ValueError("scales is empty")
    if n and L.debug_checks():   # a host sync; the kernel clamps out-of-range indices otherwise
        lo_i, hi_i = (int(v) for v in torch.aminmax(hi))
        if lo_i < 0 or hi_i >= sc.numel():
            raise ValueError(f"head_indices must lie in [0, {sc.numel()}), got [{lo_i}, {hi_i}]")
    out = torch.empty(n, 8, dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        L.check(L.lib().lq_unpack_compact(p.data_ptr(), bits_per_dim, n, sc.data_ptr(), sc.numel(), hi.data_ptr(),
                                          out.data_ptr(), L.stream_ptr(dev)), "lq_unpack_compact")
    return out
