"""Fixed-rate E8 storage on gfx950 (API of reference core/compact_storage.py).

Layout (core/compact_storage.py:87-154): one big-endian b-byte word per
vector, b in {3, 4, 5}: [coset (1) | c0..c6 (b bits each) | c7 >> 1 (b - 1)],
coordinates biased by R = 2^(b-1).  The low bit of c7 is recovered from the
even-sum constraint (floor-mod parity of c0 + .. + c6).

validate / pack / unpack run in lq_e8_validate, lq_pack_compact and
lq_unpack_e8.  Strict errors are kept: pack_e8 raises ValueError on invalid
or out-of-range points (core/compact_storage.py:112, :130).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import torch

from .. import _lib as L
from .._dev import back, to_gpu


def _flags(q: torch.Tensor, bits: int = 0, atol: float = 1e-5) -> torch.Tensor:
    qg = to_gpu(q, torch.float32).view(-1, 8)
    f = torch.empty(qg.shape[0], dtype=torch.int32, device=qg.device)
    L.check(L.lib().lq_e8_validate(qg.data_ptr(), qg.shape[0], float(atol), int(bits), f.data_ptr(),
                                   L.stream_ptr(qg.device)), "lq_e8_validate")
    return f


def validate_e8(q: torch.Tensor, atol: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """(is_valid (N,) bool, coset (N,) long): consistently integer or
    half-integer within atol, with an even integer sum.  core/compact_storage.py:39-80"""
    f = _flags(q, 0, atol)
    return back((f & L.LQ_V_VALID) != 0, q), back(((f & L.LQ_V_HALF) != 0).long(), q)


def representable_range(bits_per_dim: int) -> Tuple[int, int]:
    """core/compact_storage.py:229-232"""
    R = 2 ** (bits_per_dim - 1)
    return -R, R - 1


def check_representable(q: torch.Tensor, bits_per_dim: int) -> torch.Tensor:
    """Valid E8 points whose integer coordinates fit in [-R, R-1].  core/compact_storage.py:235-249"""
    f = _flags(q, bits_per_dim)
    return back((f & L.LQ_V_INRANGE) != 0, q)


def pack_e8(q: torch.Tensor, bits_per_dim: int) -> torch.Tensor:
    """(N, 8) valid in-range E8 points -> (N, b) uint8.  core/compact_storage.py:87-154"""
    assert bits_per_dim in (3, 4, 5), f"Only integer bit rates 3,4,5 supported, got {bits_per_dim}"
    assert q.shape[-1] == 8, f"Expected 8-dim vectors, got {q.shape[-1]}"
    qg = to_gpu(q, torch.float32).view(-1, 8)
    n = qg.shape[0]
    f = _flags(qg, bits_per_dim)
    n_invalid = int(((f & L.LQ_V_VALID) == 0).sum().item())
    if n_invalid > 0:
        raise ValueError(f"{n_invalid}/{n} inputs are not valid E₈ points. All coordinates must be consistently "
                         "integer or half-integer with even sum on the integer representation.")
    n_oor = int(((f & L.LQ_V_INRANGE) == 0).sum().item())
    if n_oor > 0:
        lo, hi = representable_range(bits_per_dim)
        raise ValueError(f"{n_oor}/{n} vectors have coordinates outside [{lo}, {hi}]. At {bits_per_dim} bits/dim, "
                         f"lattice coordinates must fit in {bits_per_dim}-bit signed range.")
    out = torch.empty(n, bits_per_dim, dtype=torch.uint8, device=qg.device)
    ok = torch.empty(n, dtype=torch.int32, device=qg.device)
    L.check(L.lib().lq_pack_compact(qg.data_ptr(), bits_per_dim, n, out.data_ptr(), ok.data_ptr(),
                                    L.stream_ptr(qg.device)), "lq_pack_compact")
    return back(out, q)


def unpack_e8(packed_bytes: torch.Tensor, bits_per_dim: int) -> torch.Tensor:
    """(N, b) uint8 -> (N, 8) fp32 E8 points.  core/compact_storage.py:157-222"""
    assert bits_per_dim in (3, 4, 5)
    assert packed_bytes.dtype == torch.uint8
    assert packed_bytes.ndim == 2
    assert packed_bytes.shape[1] == bits_per_dim, \
        f"Expected {bits_per_dim} bytes per vector, got {packed_bytes.shape[1]}"
    pg = to_gpu(packed_bytes)
    n = pg.shape[0]
    q = torch.empty(n, 8, dtype=torch.float32, device=pg.device)
    L.check(L.lib().lq_unpack_e8(pg.data_ptr(), bits_per_dim, n, q.data_ptr(), L.stream_ptr(pg.device)),
            "lq_unpack_e8")
    return back(q, packed_bytes)


def _int_to_bytes(packed_int: torch.Tensor, num_bytes: int, device) -> torch.Tensor:
    """Big-endian bytes of an int64 tensor (core/compact_storage.py:256-264)."""
    out = torch.empty(packed_int.shape[0], num_bytes, dtype=torch.uint8, device=device)
    t = packed_int.to(device)
    for i in range(num_bytes - 1, -1, -1):
        out[:, i] = (t & 0xFF).to(torch.uint8)
        t = t >> 8
    return out


def _bytes_to_int(byte_tensor: torch.Tensor, device) -> torch.Tensor:
    """Inverse of _int_to_bytes (core/compact_storage.py:267-272)."""
    r = torch.zeros(byte_tensor.shape[0], dtype=torch.int64, device=device)
    for i in range(byte_tensor.shape[1]):
        r = (r << 8) | byte_tensor[:, i].to(device).long()
    return r


@dataclass
class CompactE8Tensor:
    """Packed E8 vectors + per-group scales (core/compact_storage.py:279-331)."""
    packed: torch.Tensor
    scales: torch.Tensor
    bits_per_dim: int
    orig_shape: tuple
    group_size: int
    num_vectors: int

    @property
    def packed_bytes(self) -> int:
        return self.packed.nelement() * self.packed.element_size()

    @property
    def scale_bytes(self) -> int:
        return self.scales.nelement() * self.scales.element_size()

    @property
    def total_bytes(self) -> int:
        return self.packed_bytes + self.scale_bytes

    @property
    def fp16_bytes(self) -> int:
        return self.num_vectors * 8 * 2

    @property
    def effective_bits_per_dim(self) -> float:
        return (self.total_bytes * 8) / (self.num_vectors * 8)

    @property
    def compression_ratio(self) -> float:
        return self.fp16_bytes / self.total_bytes

    def summary(self) -> str:
        return "\n".join([
            "CompactE8Tensor (theoretical storage)",
            f"  Vectors: {self.num_vectors:,} x 8-dim",
            f"  Nominal rate: {self.bits_per_dim} bits/dim",
            f"  Effective rate: {self.effective_bits_per_dim:.3f} bits/dim (incl. scales)",
            f"  Packed: {self.packed_bytes:,} B | Scales: {self.scale_bytes:,} B | Total: {self.total_bytes:,} B",
            f"  FP16 equiv: {self.fp16_bytes:,} B | Compression: {self.compression_ratio:.2f}x",
        ])


def quantize_and_pack(x: torch.Tensor, bits_per_dim: int, scale: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """encode_e8(x / scale), then pack the representable vectors.
    Returns (packed (M, b) uint8, in_range (N,) bool).  core/compact_storage.py:338-360"""
    from .e8_quantizer import encode_e8
    q = encode_e8(to_gpu(x, torch.float32).view(-1, 8) / scale)
    in_range = check_representable(q, bits_per_dim)
    if int(in_range.sum().item()) == 0:
        return back(torch.zeros(0, bits_per_dim, dtype=torch.uint8, device=q.device), x), back(in_range, x)
    packed = pack_e8(q[in_range], bits_per_dim)
    return back(packed, x), back(in_range, x)


def unpack_and_dequantize(packed: torch.Tensor, bits_per_dim: int, scale: float) -> torch.Tensor:
    """unpack_e8(packed) * scale.  core/compact_storage.py:363-370"""
    return unpack_e8(packed, bits_per_dim) * scale
