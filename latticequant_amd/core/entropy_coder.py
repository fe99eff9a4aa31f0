"""Parity-aware symbolisation of E8 points (API of reference core/entropy_coder.py:46-89).

An E8 point is (coset bit, 7 free integer coordinates, floor(c7 / 2)); the
low bit of c7 follows from the even-sum constraint.  Both directions run in
the lq_e8_to_symbols / lq_symbols_to_e8 kernels.
"""
from __future__ import annotations

import torch

from .. import _lib as L
from .._dev import back, to_gpu


def e8_to_symbols(q: torch.Tensor):
    """E8 point (N, 8) -> (coset (N,), free (N, 7), coord8_half (N,)), int64.
    core/entropy_coder.py:46-68"""
    qg = to_gpu(q, torch.float32).view(-1, 8)
    n = qg.shape[0]
    cos = torch.empty(n, dtype=torch.int32, device=qg.device)
    sym = torch.empty(n, 8, dtype=torch.int32, device=qg.device)
    L.check(L.lib().lq_e8_to_symbols(qg.data_ptr(), n, cos.data_ptr(), sym.data_ptr(), L.stream_ptr(qg.device)),
            "lq_e8_to_symbols")
    sym = sym.long()
    return back(cos.long(), q), back(sym[:, :7].contiguous(), q), back(sym[:, 7].contiguous(), q)


def symbols_to_e8(coset: torch.Tensor, free_coords: torch.Tensor, coord8_half: torch.Tensor) -> torch.Tensor:
    """Inverse of e8_to_symbols (lossless).  core/entropy_coder.py:71-89"""
    c = to_gpu(coset, torch.int32).view(-1)
    n = c.shape[0]
    sym = torch.empty(n, 8, dtype=torch.int32, device=c.device)
    sym[:, :7] = to_gpu(free_coords, torch.int32).view(n, 7)
    sym[:, 7] = to_gpu(coord8_half, torch.int32).view(n)
    out = torch.empty(n, 8, dtype=torch.float32, device=c.device)
    L.check(L.lib().lq_symbols_to_e8(c.data_ptr(), sym.data_ptr(), n, out.data_ptr(), L.stream_ptr(c.device)),
            "lq_symbols_to_e8")
    return back(out, coset)
