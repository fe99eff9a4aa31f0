"""The reference's CPU write / read path "as written": torch-CPU tensor ops for
the E8 search, symbols and scales, and per-symbol Python loops for the rANS
table normalisation, encode and decode -- the structure of
core/e8_quantizer.py:20-83, core/entropy_coder.py:46-89,
core/gpu_ans.py:62-168 and llm/compressed_kv_cache.py:176-332 -- restated here
so bench.py can time the reference's own CPU cost beside the GPU (the C oracle
in lq_oracle.c is the fast restatement).

Test / baseline infrastructure only: it is the cpu_baseline "as written" tier
of bench.py and is checked against the C oracle in tests/test_oracle.py
(identical bitstreams and decoded values); nothing in latticequant_amd uses it.
"""
from __future__ import annotations

import numpy as np
import torch

from . import oracle as O

L, LOG2_L = 1024, 10


def d8_torch(x: torch.Tensor) -> torch.Tensor:
    """Nearest D8 point with the reference's fp32 decisions, in torch CPU ops
    (core/e8_quantizer.py:20-58)."""
    r = torch.round(x)
    odd = (r.sum(-1) % 2) != 0
    res = x - r
    cost = (1 - 2 * res.abs()) + torch.arange(8, dtype=x.dtype) * 1e-7
    k = cost.argmin(-1)
    rows = torch.nonzero(odd).squeeze(-1)
    if rows.numel():
        cols = k[rows]
        sg = torch.sign(res[rows, cols])
        r[rows, cols] += torch.where(sg == 0, torch.ones_like(sg), sg)
    return r


def e8_torch(x: torch.Tensor) -> torch.Tensor:
    """Nearest E8 point, torch CPU (core/e8_quantizer.py:61-83)."""
    c1 = d8_torch(x)
    c2 = d8_torch(x - 0.5) + 0.5
    use1 = ((x - c1) ** 2).sum(-1) <= ((x - c2) ** 2).sum(-1)
    return torch.where(use1.unsqueeze(-1), c1, c2)


def normalise(counts: np.ndarray) -> np.ndarray:
    """build_rans_table's frequencies (core/gpu_ans.py:62-98): one Python pass
    per adjustment round, numpy's argsort order (the restated tie rule of the
    oracle)."""
    return O._normalise_numpy(counts.astype(np.int64))


def encode_stream(col: np.ndarray, lo: int, freqs: np.ndarray):
    """rANS encode of one stream, one Python iteration per symbol and per
    renormalisation bit (core/gpu_ans.py:105-139); returns (words, state, n_bits)."""
    cum = np.concatenate([[0], np.cumsum(freqs)]).tolist()
    f = freqs.tolist()
    out = []
    x = L
    for v in col[::-1].tolist():
        s = v - lo
        fs, cs = f[s], cum[s]
        while x >= 2 * fs:
            out.append(x & 1)
            x >>= 1
        x = (x // fs) * L + cs + x % fs
    out.reverse()
    n = len(out)
    words = [0] * ((n + 31) // 32 + 1)
    for i, b in enumerate(out):
        if b:
            words[i >> 5] |= 1 << (i & 31)
    return np.array(words, dtype=np.uint32), x, n


def decode_stream(words: np.ndarray, n_bits: int, state: int, lo: int, freqs: np.ndarray, n: int) -> np.ndarray:
    """rANS decode, one Python iteration per symbol and bit (core/gpu_ans.py:146-168)."""
    cum = np.concatenate([[0], np.cumsum(freqs)]).tolist()
    slot_sym = np.repeat(np.arange(len(freqs)), freqs).tolist()
    f = freqs.tolist()
    w = words.tolist()
    out = [0] * n
    x, p = state, 0
    for i in range(n):
        slot = x & (L - 1)
        s = slot_sym[slot]
        out[i] = s + lo
        x = f[s] * (x >> LOG2_L) + slot - cum[s]
        while x < L and p < n_bits:
            x = (x << 1) | ((w[p >> 5] >> (p & 31)) & 1)
            p += 1
    return np.array(out, dtype=np.int64)


def compress(t: torch.Tensor, bits: int, scales_f32=None):
    """One _compress_tensor call on a CPU tensor (B, H, T, hd): scales, E8,
    symbols, per (coset, coordinate) table + stream.  Returns (streams,
    scale16) with streams = [(coset, idx, words, state, n_bits, lo, freqs, n)]."""
    B, H, T, hd = t.shape
    th = t.float().reshape(B * H, -1, 8)
    if scales_f32 is None:
        s2 = (th ** 2).mean(dim=(1, 2))
        sc = (2 * torch.pi * torch.e * s2 * 4.0 ** (-bits)).sqrt()
        sc = torch.where(s2 < 1e-12, torch.ones_like(sc), sc)
    else:
        sc = torch.as_tensor(scales_f32, dtype=torch.float32)
    q = e8_torch((th / sc[:, None, None]).reshape(-1, 8))
    coset = (q[:, 0] - q[:, 0].round()).abs() > 0.25
    ic = (q - 0.5 * coset[:, None]).round().to(torch.int64)
    syms = torch.cat([ic[:, :7], torch.div(ic[:, 7], 2, rounding_mode="floor")[:, None]], 1).numpy()
    cos = coset.numpy()
    streams = []
    for c in (0, 1):
        sc_rows = syms[cos == c]
        if not len(sc_rows):
            continue
        for i in range(8):
            col = sc_rows[:, i]
            lo = int(col.min()) - 2
            counts = np.bincount(col - lo, minlength=int(col.max()) + 3 - lo)
            freqs = normalise(counts)
            words, state, nb = encode_stream(col, lo, freqs)
            streams.append((c, i, words, state, nb, lo, freqs, len(col)))
    return streams, sc.to(torch.float16), cos


def decompress(streams, cos: np.ndarray, scale16: torch.Tensor, shape) -> np.ndarray:
    """_decompress_chunk on the CPU: decode every stream, rebuild c7 from the
    parity of the free coordinates, x fp16 scale per head (llm/compressed_kv_cache.py:289-332)."""
    n = len(cos)
    sym = np.zeros((n, 8), np.int64)
    for c, i, words, state, nb, lo, freqs, cnt in streams:
        sym[cos == c, i] = decode_stream(words, nb, state, lo, freqs, cnt)
    c7 = 2 * sym[:, 7] + np.mod(sym[:, :7].sum(1), 2)
    q = np.concatenate([sym[:, :7], c7[:, None]], 1).astype(np.float32) + 0.5 * cos[:, None].astype(np.float32)
    B, H, T, hd = shape
    s = scale16.float().numpy()
    out = q.reshape(B * H, -1, 8) * s[:, None, None]
    return out.reshape(shape).astype(np.float16)
