"""Randomized Hadamard transform (API of reference core/pipeline.py:33-118 and
llm/perplexity_eval.py:35-61 HeadRHT).

w = (1/sqrt(d)) H D_eps v with Sylvester H and random signs eps.  The signs
come from torch's CPU generator exactly as the reference draws them
(rand(d) < 0.5 -> +1, else -1), so they are the reference's bit for bit; the
transform itself runs in lq_rht (fp32, reference butterfly order, then one
IEEE division by f32(sqrt(d))).
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .._dev import back, to_gpu


def hadamard_matrix(n: int) -> torch.Tensor:
    """Unnormalised Sylvester Hadamard matrix (core/pipeline.py:33-46)."""
    assert n > 0 and (n & (n - 1)) == 0, f"n must be power of 2, got {n}"
    H = torch.tensor([[1.0]])
    while H.shape[0] < n:
        H = torch.cat([torch.cat([H, H], dim=1), torch.cat([H, -H], dim=1)], dim=0)
    return H


def sign_vector(d: int, seed: int) -> torch.Tensor:
    """Random +-1 signs of RHT(d, seed) (core/pipeline.py:93-98), CPU fp32."""
    gen = torch.Generator()
    gen.manual_seed(int(seed))
    return torch.where(torch.rand(d, generator=gen) < 0.5, torch.ones(d), -torch.ones(d))


def _rht(x: torch.Tensor, signs: torch.Tensor, inverse: bool, rows_per_sign: int = 0,
         out_dtype=None) -> torch.Tensor:
    d = x.shape[-1]
    if d < 8 or d > 512 or d & (d - 1):
        raise ValueError(f"lq_rht handles power-of-two d in [8, 512], got {d}")
    xg = to_gpu(x)
    if xg.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        xg = xg.float()
    n_rows = xg.numel() // d
    sg = signs.to(device=xg.device, dtype=torch.float32).contiguous().view(-1, d)
    od = out_dtype or torch.float32
    out = torch.empty(xg.shape, dtype=od, device=xg.device)
    L.check(L.lib().lq_rht(xg.data_ptr(), L.dtype_code(xg.dtype), n_rows, d, sg.data_ptr(),
                           rows_per_sign if rows_per_sign > 0 else max(n_rows, 1), sg.shape[0], 1 if inverse else 0,
                           out.data_ptr(), L.dtype_code(od), L.stream_ptr(xg.device)), "lq_rht")
    return back(out, x)


def fast_hadamard_transform(x: torch.Tensor) -> torch.Tensor:
    """H x / sqrt(d) over the last dim, fp32 (core/pipeline.py:49-69)."""
    d = x.shape[-1]
    return _rht(x, torch.ones(d), inverse=False)


def inverse_fast_hadamard_transform(x: torch.Tensor) -> torch.Tensor:
    """Self-inverse: the same transform (core/pipeline.py:72-78)."""
    return fast_hadamard_transform(x)


class RHT:
    """Randomized Hadamard Transform with seeded signs (core/pipeline.py:81-118)."""

    def __init__(self, d: int, seed: int = 0):
        assert d % 8 == 0, f"d must be divisible by 8, got {d}"
        self.d = d
        self.signs = sign_vector(d, seed)

    def forward(self, v: torch.Tensor) -> torch.Tensor:
        """v -> (1/sqrt(d)) H D_eps v"""
        return _rht(v, self.signs, inverse=False)

    def inverse(self, w: torch.Tensor) -> torch.Tensor:
        """w -> D_eps (1/sqrt(d)) H w"""
        return _rht(w, self.signs, inverse=True)


class HeadRHT:
    """Per (layer, head, K/V) RHT, seed layer*10000 + head*10 + kv (llm/perplexity_eval.py:35-61)."""

    def __init__(self, head_dim: int, layer_idx: int, head_idx: int, kv_type: int):
        self.seed = layer_idx * 10000 + head_idx * 10 + kv_type
        self.signs = sign_vector(head_dim, self.seed)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _rht(x, self.signs, inverse=False)

    def inverse(self, x: torch.Tensor) -> torch.Tensor:
        return _rht(x, self.signs, inverse=True)


def head_signs(head_dim: int, layer_idx: int, n_heads: int, kv_type: int) -> torch.Tensor:
    """(n_heads, head_dim) HeadRHT sign rows of one layer and K/V."""
    return torch.stack([sign_vector(head_dim, layer_idx * 10000 + h * 10 + kv_type) for h in range(n_heads)])


def rht_heads(x: torch.Tensor, signs: torch.Tensor, inverse: bool = False, out_dtype=None) -> torch.Tensor:
    """Batched HeadRHT over a (B, H, T, d) tensor with (H, d) sign rows in one launch."""
    if x.dim() != 4 or signs.shape != (x.shape[1], x.shape[3]):
        raise ValueError("x must be (B, H, T, d) and signs (H, d)")
    return _rht(x, signs, inverse=inverse, rows_per_sign=x.shape[2], out_dtype=out_dtype)
