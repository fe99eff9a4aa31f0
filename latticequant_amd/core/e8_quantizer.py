"""E8 lattice quantizer on gfx950 (API of reference core/e8_quantizer.py).

E8 = D8 u (D8 + 1/2), D8 = {z in Z^8 : sum(z) even}.  The nearest point is
found with the Conway-Sloane decoder: nearest D8 point of x and of x - 1/2,
keep the closer.  The kernel (lq_e8_encode_f32) reproduces the reference's
fp32 rounding: half-to-even rounding, flip cost RN(RN(1 - 2|r|) + i*1e-7)
with first-index argmin, and squared distances summed left to right.

Inputs on the CPU are moved to the current ROCm device and the result is
returned on the input's device; a GPU is required.
"""
from __future__ import annotations

import numpy as np
import torch

from .. import _lib as L
from .._dev import back, to_gpu

G_E8 = 0.0717          # normalised second moment of E8 (core/e8_quantizer.py:131)
VOL_E8_UNIT = 1.0


def _encode(x: torch.Tensor, mode: int) -> torch.Tensor:
    if x.shape[-1] != 8:
        raise ValueError(f"expected (N, 8), got {tuple(x.shape)}")
    xg = to_gpu(x, torch.float32).view(-1, 8)
    out = torch.empty_like(xg)
    L.check(L.lib().lq_e8_encode_f32(xg.data_ptr(), xg.shape[0], mode, out.data_ptr(), L.stream_ptr(xg.device)),
            "lq_e8_encode_f32")
    return back(out.view(x.shape), x)


def encode_d8(x: torch.Tensor) -> torch.Tensor:
    """Nearest D8 point of each row of x (N, 8).  core/e8_quantizer.py:20-58"""
    return _encode(x, 1)


def encode_e8(x: torch.Tensor) -> torch.Tensor:
    """Nearest E8 point of each row of x (N, 8).  core/e8_quantizer.py:61-83"""
    return _encode(x, 0)


def quantize_e8(x: torch.Tensor, scale: float) -> torch.Tensor:
    """x -> Q_E8(x / scale) * scale for any (..., 8) tensor.  core/e8_quantizer.py:90-110"""
    orig_shape = x.shape
    xf = to_gpu(x, torch.float32).reshape(-1, 8)
    q = encode_e8(xf / scale)
    return back((q * scale).reshape(orig_shape), x)


def dequantize_error(x: torch.Tensor, x_hat: torch.Tensor) -> dict:
    """Per-dimension MSE and max error.  core/e8_quantizer.py:113-123"""
    err = x - x_hat
    mse = (err ** 2).mean().item()
    return {"mse_per_dim": (err ** 2).reshape(-1, 8).mean().item(), "mse_total": mse,
            "max_abs_err": err.abs().max().item()}


def compute_scale(sigma2: float, bits_per_dim: float) -> float:
    """Lattice scale a = sqrt(2 pi e sigma^2 4^-b) (Theorem 2).  core/e8_quantizer.py:137-148"""
    target_vol_2n = 2 * np.pi * np.e * sigma2 * (4 ** (-bits_per_dim))
    return np.sqrt(target_vol_2n)


def theoretical_mse(sigma2: float, bits_per_dim: float) -> float:
    """D = G(E8) 2 pi e sigma^2 4^-b per dimension.  core/e8_quantizer.py:151-156"""
    return G_E8 * 2 * np.pi * np.e * sigma2 * (4 ** (-bits_per_dim))
