"""CPU oracle for the LatticeQuant compressed-KV hot path.

TEST INFRASTRUCTURE ONLY.  This module is the checker that the HIP path is
compared against.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py may import it; the product package
(latticequant_amd) never does.

It restates the reference algorithm (yoon9728/LatticeQuant) in numpy on top of
the plain-C kernels in lq_oracle.c.  Each function names the reference
file:line it follows.  Pinning is described in lq_oracle.c; everything here
is additionally checked against the golden vectors under tests/golden/,
which were written by the reference itself, and against closed forms,
brute force and invariants (tests/test_oracle.py).

Parity notes
  * torch.round is round-half-even, argmin takes the first index, torch's CPU
    sum over an 8-wide row runs left to right: all restated exactly.
  * numpy.argsort tie order (used by build_rans_table) is restated for n <= 256
    as numpy's AVX512 bitonic network.  For n > 256 this module calls the host
    numpy.argsort, so on a host whose numpy takes another code path the tie
    order there is "parity unpinned".
  * escape_shifts / compress_chunk(escape=True) / decompress_chunk: the
    coarse / fine escape for alphabets beyond L is a format of this build
    (the reference's normalisation never terminates there), so its parity is
    unpinned by the reference; it is pinned by invariants instead (lossless
    round trip, coarse alphabets within L, minimal shift) in
    tests/test_oracle.py.
  * sigma^2 = mean(x^2) is reduction-order dependent in the reference; the
    oracle computes it in float64 and rounds once.  Bit-exact comparisons inject
    the scale instead.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

L = 1024
LOG2_L = 10
HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(HERE, "_build", "liblq_oracle.so")
_lib = None


def build() -> str:
    """Compile lq_oracle.c into oracle/_build/liblq_oracle.so."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO) or os.path.getmtime(_SO) < os.path.getmtime(os.path.join(HERE, "lq_oracle.c")):
            build()
        _lib = ctypes.CDLL(_SO)
        i64, i32, f32p = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        for name, args, res in [
            ("lqo_encode_d8", [f32p, f32p, i64], None),
            ("lqo_encode_e8", [f32p, f32p, i64], None),
            ("lqo_quantize_heads", [f32p, f32p, i64, i64, f32p], None),
            ("lqo_quantize_heads_dither", [f32p, f32p, i64, i64, i64, f32p], None),
            ("lqo_dither", [i64, i64, i64, f32p], None),
            ("lqo_mix64", [ctypes.c_uint64], ctypes.c_uint64),
            ("lqo_e8_to_symbols", [f32p, i64, f32p, f32p], None),
            ("lqo_symbols_to_e8", [f32p, f32p, i64, f32p], None),
            ("lqo_pack_coset_bits", [f32p, i64, f32p], None),
            ("lqo_pack_e8", [f32p, i64, i32, f32p], ctypes.c_int),
            ("lqo_unpack_e8", [f32p, i64, i32, f32p], None),
            ("lqo_argsort", [f32p, i32, i64, f32p], ctypes.c_int),
            ("lqo_build_table", [f32p, i32, f32p], ctypes.c_int),
            ("lqo_table_lookup", [f32p, i32, f32p, f32p], None),
            ("lqo_rans_encode", [f32p, i64, f32p, f32p, f32p, i64, f32p, f32p], ctypes.c_int64),
            ("lqo_rans_decode", [f32p, i64, i64, f32p, f32p, f32p, i64, f32p], None),
        ]:
            fn = getattr(_lib, name)
            fn.argtypes = args
            fn.restype = res
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ E8 ---

def encode_d8(x: np.ndarray) -> np.ndarray:
    """core/e8_quantizer.py:20-58"""
    x = _c(x, np.float32).reshape(-1, 8)
    out = np.empty_like(x)
    lib().lqo_encode_d8(_p(x), _p(out), x.shape[0])
    return out


def encode_e8(x: np.ndarray) -> np.ndarray:
    """core/e8_quantizer.py:61-83"""
    x = _c(x, np.float32).reshape(-1, 8)
    out = np.empty_like(x)
    lib().lqo_encode_e8(_p(x), _p(out), x.shape[0])
    return out


def compute_scale(sigma2: float, bits_per_dim: float) -> float:
    """core/e8_quantizer.py:137-148 (float64 scalar form)."""
    return float(np.sqrt(2 * np.pi * np.e * sigma2 * (4 ** (-bits_per_dim))))


def cache_scales(sigma2_f32: np.ndarray, bits: int):
    """Vectorised per-head scale of _compress_tensor (llm/compressed_kv_cache.py:192-196):
    RN32(RN32(2*pi*e) * sigma2) * 4^-b, sqrt, sigma2 < 1e-12 -> 1, fp16 copy."""
    s2 = _c(sigma2_f32, np.float32)
    c = np.float32(2 * math.pi * math.e)
    tv = (c * s2).astype(np.float32) * np.float32(4.0 ** (-bits))
    sc = np.sqrt(tv.astype(np.float32)).astype(np.float32)
    sc = np.where(s2 < np.float32(1e-12), np.float32(1.0), sc).astype(np.float32)
    return sc, sc.astype(np.float16)


def head_sigma2(t: np.ndarray) -> np.ndarray:
    """mean(t^2) per head (llm/compressed_kv_cache.py:189), float64 accumulate, one rounding."""
    th = np.asarray(t, dtype=np.float64).reshape(t.shape[0] * t.shape[1], -1)
    return (th * th).mean(axis=1).astype(np.float32)


def quantize_heads(t32: np.ndarray, scales: np.ndarray, dither_seed: Optional[int] = None) -> np.ndarray:
    """x / scale[head] then encode_e8 (llm/compressed_kv_cache.py:199-201);
    with dither_seed, x / scale + dither (build-defined, see dither())."""
    t32 = _c(t32, np.float32)
    nh = scales.shape[0]
    bph = t32.size // (8 * nh)
    sc = _c(scales, np.float32)
    q = np.empty((nh * bph, 8), dtype=np.float32)
    if dither_seed is None:
        lib().lqo_quantize_heads(_p(t32), _p(sc), nh, bph, _p(q))
    else:
        lib().lqo_quantize_heads_dither(_p(t32), _p(sc), nh, bph, int(dither_seed), _p(q))
    return q


def dither(seed: int, n_vectors: int, v0: int = 0) -> np.ndarray:
    """Subtractive dither of vectors v0 .. v0+n-1 of a chunk: (n, 8) float32 in
    [-1, 1) (build-defined; lq_oracle.c lqo_dither)."""
    d = np.empty((n_vectors, 8), dtype=np.float32)
    lib().lqo_dither(int(seed), int(v0), int(n_vectors), _p(d))
    return d


def e8_to_symbols(q: np.ndarray):
    """core/entropy_coder.py:46-68 -> (coset (N,), free (N,7), c8h (N,))"""
    q = _c(q, np.float32).reshape(-1, 8)
    n = q.shape[0]
    cos = np.empty(n, dtype=np.int32)
    sym = np.empty((n, 8), dtype=np.int32)
    lib().lqo_e8_to_symbols(_p(q), n, _p(cos), _p(sym))
    return cos.astype(np.int64), sym[:, :7].astype(np.int64), sym[:, 7].astype(np.int64)


def symbols_to_e8(coset, free, c8h) -> np.ndarray:
    """core/entropy_coder.py:71-89"""
    n = len(coset)
    cos = _c(coset, np.int32)
    sym = np.empty((n, 8), dtype=np.int32)
    sym[:, :7] = free
    sym[:, 7] = c8h
    q = np.empty((n, 8), dtype=np.float32)
    lib().lqo_symbols_to_e8(_p(cos), _p(sym), n, _p(q))
    return q


def pack_coset_bits(coset) -> np.ndarray:
    """llm/compressed_kv_cache.py:46-54"""
    cos = _c(coset, np.int32)
    out = np.zeros((len(cos) + 7) // 8, dtype=np.uint8)
    lib().lqo_pack_coset_bits(_p(cos), len(cos), _p(out))
    return out


def unpack_coset_bits(packed: np.ndarray, n: int) -> np.ndarray:
    """llm/compressed_kv_cache.py:57-63"""
    i = np.arange(n)
    return ((np.asarray(packed, np.uint8)[i // 8] >> (i % 8)) & 1).astype(np.uint8)


# ------------------------------------------------------- compact storage ---

def validate_e8(q: np.ndarray, atol: float = 1e-5):
    """core/compact_storage.py:39-80 -> (is_valid, coset)"""
    q = np.asarray(q, dtype=np.float32)
    is_int = np.abs(q - np.round(q)).max(-1) < atol
    h = q - np.float32(0.5)
    is_half = np.abs(h - np.round(h)).max(-1) < atol
    ic = np.where(is_half[:, None], h, q)
    ic = np.round(ic).astype(np.int64)
    even = (ic.sum(-1) % 2) == 0
    return (is_int | is_half) & even, is_half.astype(np.int64)


def check_representable(q: np.ndarray, bits: int) -> np.ndarray:
    """core/compact_storage.py:235-249"""
    valid, coset = validate_e8(q)
    qq = np.asarray(q, np.float32)
    ic = np.round(np.where(coset[:, None] == 1, qq - np.float32(0.5), qq)).astype(np.int64)
    R = 2 ** (bits - 1)
    return valid & (ic >= -R).all(-1) & (ic <= R - 1).all(-1)


def pack_e8(q: np.ndarray, bits: int) -> np.ndarray:
    """core/compact_storage.py:87-154 (strict: ValueError on invalid / out of range)"""
    q = _c(q, np.float32).reshape(-1, 8)
    valid, _ = validate_e8(q)
    if (~valid).any():
        raise ValueError(f"{int((~valid).sum())}/{len(q)} inputs are not valid E8 points")
    out = np.empty((q.shape[0], bits), dtype=np.uint8)
    if lib().lqo_pack_e8(_p(q), q.shape[0], bits, _p(out)) != 0:
        raise ValueError("coordinates outside the representable range")
    return out


def unpack_e8(packed: np.ndarray, bits: int) -> np.ndarray:
    """core/compact_storage.py:157-222"""
    packed = _c(packed, np.uint8)
    n = packed.shape[0]
    q = np.empty((n, 8), dtype=np.float32)
    lib().lqo_unpack_e8(_p(packed), n, bits, _p(q))
    return q


# ---------------------------------------------------------------- rANS ---

def argsort(keys: np.ndarray, pad: int) -> np.ndarray:
    """numpy.argsort tie order restated (n <= 256), else host numpy."""
    k = _c(keys, np.int64)
    n = len(k)
    out = np.empty(n, dtype=np.int32)
    if lib().lqo_argsort(_p(k), n, int(pad), _p(out)) != 0:
        return np.argsort(np.asarray(keys)).astype(np.int32)
    return out


@dataclass
class Table:
    freqs: np.ndarray
    cumfreqs: np.ndarray
    lookup: np.ndarray
    alphabet: List[int]
    n_symbols: int


def _normalise_numpy(counts: np.ndarray) -> np.ndarray:
    """The core/gpu_ans.py:62-86 loop with host numpy.argsort (used for n > 256)."""
    n = len(counts)
    total = counts.sum()
    freqs = np.ones(n, np.int32) if total == 0 else np.maximum((counts / total * L).astype(np.int32), 1)
    while freqs.sum() != L:
        diff = L - freqs.sum()
        if diff > 0:
            order = np.argsort(-counts)
            for j in range(abs(diff)):
                freqs[order[j % n]] += 1
        else:
            order = np.argsort(-freqs)
            for j in range(abs(diff)):
                idx = order[j % n]
                if freqs[idx] > 1:
                    freqs[idx] -= 1
    return freqs


def build_rans_table(counts: np.ndarray, alphabet: List[int]) -> Table:
    """core/gpu_ans.py:62-98"""
    c = _c(counts, np.int64)
    n = len(alphabet)
    if n > L:
        raise ValueError(f"alphabet of {n} symbols exceeds L={L}; the reference never terminates here")
    freqs = np.empty(n, dtype=np.int32)
    rc = lib().lqo_build_table(_p(c), n, _p(freqs))
    if rc == -2:
        freqs = _normalise_numpy(c.copy())
    elif rc != 0:
        raise ValueError(f"build_rans_table failed ({rc})")
    cum = np.empty(n + 1, dtype=np.int32)
    lookup = np.empty(L, dtype=np.int32)
    lib().lqo_table_lookup(_p(freqs), n, _p(cum), _p(lookup))
    return Table(freqs=freqs, cumfreqs=cum, lookup=lookup, alphabet=list(alphabet), n_symbols=n)


def symbol_indices(symbols: np.ndarray, alphabet: List[int]) -> np.ndarray:
    """Symbol -> table index as rans_encode resolves it (core/gpu_ans.py:110-119):
    exact match (last duplicate wins, as a dict does) else the first nearest entry."""
    alph = np.asarray(alphabet, dtype=np.int64)
    lut = {int(v): i for i, v in enumerate(alph)}
    s = np.asarray(symbols, dtype=np.int64)
    out = np.empty(len(s), dtype=np.int32)
    for u in np.unique(s):
        i = lut.get(int(u))
        if i is None:
            i = int(np.argmin(np.abs(alph - u)))
        out[s == u] = i
    return out


def rans_encode(symbols: np.ndarray, table: Table):
    """core/gpu_ans.py:105-139 -> (uint32 words incl. trailing zero word, state, n_bits)"""
    idx = symbol_indices(symbols, table.alphabet)
    n = len(idx)
    max_words = (10 * n + 31) // 32 + 2
    words = np.zeros(max_words, dtype=np.uint32)
    st = np.zeros(1, np.int64)
    nb = np.zeros(1, np.int64)
    nw = lib().lqo_rans_encode(_p(idx), n, _p(table.freqs), _p(table.cumfreqs), _p(words), max_words,
                               _p(st), _p(nb))
    assert nw > 0
    return words[:nw].copy(), int(st[0]), int(nb[0])


def rans_decode(bitstream: np.ndarray, n_bits: int, state: int, table: Table, n_symbols: int) -> np.ndarray:
    """core/gpu_ans.py:146-168 -> int64 symbol values"""
    w = _c(np.asarray(bitstream).view(np.uint32) if np.asarray(bitstream).dtype == np.int32 else bitstream,
           np.uint32)
    out = np.empty(n_symbols, dtype=np.int32)
    lib().lqo_rans_decode(_p(w), int(n_bits), int(state), _p(table.freqs), _p(table.cumfreqs),
                          _p(table.lookup), int(n_symbols), _p(out))
    alph = np.asarray(table.alphabet, dtype=np.int64)
    return alph[out]


# ----------------------------------------------------------- cache chunk ---

@dataclass
class Stream:
    coset: int
    idx: int
    n_symbols: int
    table: Table
    words: np.ndarray
    state: int
    n_bits: int


@dataclass
class Chunk:
    shape: tuple
    bits: int
    scales_f32: np.ndarray
    scales: np.ndarray            # fp16, what the chunk stores
    coset_packed: np.ndarray
    coset_counts: tuple
    streams: List[Stream] = field(default_factory=list)
    bitstream: np.ndarray = None  # merged uint32 words
    word_offsets: List[int] = field(default_factory=list)
    decompressed: np.ndarray = None
    dither_seed: Optional[int] = None
    esc_k: Optional[np.ndarray] = None   # (8,) shifts of an escaped chunk, else None
    fine: Optional[dict] = None          # coordinate j -> uint32 low-bit words (k_j > 0)

    @property
    def n_vectors(self):
        return int(np.prod(self.shape)) // 8

    @property
    def compressed_bytes(self):
        """llm/compressed_kv_cache.py:113-119 accounting (bitstream + coset bits +
        fp16 scales), plus an escaped chunk's low-bit words."""
        fine = sum(w.size for w in self.fine.values()) * 4 if self.fine else 0
        return self.bitstream.size * 4 + self.coset_packed.size + self.scales.size * 2 + fine


def column_table(col: np.ndarray):
    """Alphabet range(min-2, max+2) and counts as _compress_tensor builds them
    (llm/compressed_kv_cache.py:244-248)."""
    u, uc = np.unique(col, return_counts=True)
    lo, hi = int(u.min()) - 2, int(u.max()) + 2
    counts = np.zeros(hi - lo + 1, dtype=np.int64)
    counts[u - lo] = uc
    return lo, counts


ESC_MAX_SHIFT = 7
BLK = 512


def escape_shifts(syms: np.ndarray, coset: np.ndarray) -> np.ndarray:
    """Per coordinate j the least k in [0, 7] with (max >> k) - (min >> k) + 5 <= L
    for the symbols of both cosets' streams of j (build-defined escape; the
    reference's table normalisation never terminates beyond L)."""
    ks = np.zeros(8, np.int64)
    for j in range(8):
        for k in range(ESC_MAX_SHIFT + 1):
            ok = True
            for c in (0, 1):
                col = syms[coset == c][:, j]
                if len(col) and (int(col.max()) >> k) - (int(col.min()) >> k) + 5 > L:
                    ok = False
            if ok:
                ks[j] = k
                break
        else:
            raise ValueError(f"coordinate {j}: no shift up to {ESC_MAX_SHIFT} fits the alphabet in L")
    return ks


def pack_fine(low: np.ndarray, k: int) -> np.ndarray:
    """Low bits of every vector (value v at bit v * k, least significant first)
    in uint32 words, padded to whole 512-vector blocks (16 k words each)."""
    n = len(low)
    nblk = (n + BLK - 1) // BLK
    bits = ((np.asarray(low, np.int64)[:, None] >> np.arange(k)) & 1).astype(np.uint8).reshape(-1)
    bits = np.concatenate([bits, np.zeros(nblk * BLK * k - bits.size, np.uint8)])
    return np.packbits(bits.reshape(-1, 32), axis=1, bitorder="little").view(np.uint32).reshape(-1)


def unpack_fine(words: np.ndarray, k: int, n: int) -> np.ndarray:
    bits = np.unpackbits(np.asarray(words, np.uint32).view(np.uint8), bitorder="little")[:n * k]
    return (bits.reshape(n, k).astype(np.int64) << np.arange(k)).sum(1)


def compress_chunk(t: np.ndarray, bits: int, scales_f32: Optional[np.ndarray] = None,
                   entropy: bool = True, dither_seed: Optional[int] = None, escape: bool = False) -> Chunk:
    """CompressedKVCache._compress_tensor (llm/compressed_kv_cache.py:176-287).

    t: (B, H, T, hd) array in the model dtype.  scales_f32 injects the per-head
    fp32 scale (bit-exact comparisons); otherwise the oracle's own sigma^2.
    escape: coordinates whose alphabet exceeds L are coded as coarse symbols
    s >> k_j plus raw low bits (a format of this build; see escape_shifts)."""
    B, H, T, hd = t.shape
    assert hd % 8 == 0
    t32 = np.asarray(t, dtype=np.float32)
    nh = B * H
    if scales_f32 is None:
        sc32, sc16 = cache_scales(head_sigma2(t32), bits)
    else:
        sc32 = _c(scales_f32, np.float32)
        sc16 = sc32.astype(np.float16)
    q = quantize_heads(t32, sc32, dither_seed)
    bph = q.shape[0] // nh
    qd = q if dither_seed is None else (q - dither(dither_seed, q.shape[0])).astype(np.float32)
    dec = (qd.reshape(nh, bph, 8) * sc32[:, None, None]).astype(np.float32)
    dec = dec.reshape(t.shape).astype(np.asarray(t).dtype if np.asarray(t).dtype != np.float64 else np.float32)
    coset, free, c8h = e8_to_symbols(q)
    syms = np.concatenate([free, c8h[:, None]], 1)
    ch = Chunk(shape=t.shape, bits=bits, scales_f32=sc32, scales=sc16,
               coset_packed=pack_coset_bits(coset),
               coset_counts=(int((coset == 0).sum()), int((coset == 1).sum())), decompressed=dec,
               dither_seed=dither_seed)
    if not entropy:
        return ch
    if escape:
        ks = escape_shifts(syms, coset)
        if ks.any():
            ch.esc_k = ks
            ch.fine = {j: pack_fine(syms[:, j] & ((1 << int(ks[j])) - 1), int(ks[j])) for j in range(8) if ks[j]}
            syms = syms >> ks[None, :]
    all_words = []
    for c in (0, 1):
        sc = syms[coset == c]
        if len(sc) == 0:
            continue
        for i in range(8):
            col = sc[:, i]
            lo, counts = column_table(col)
            tab = build_rans_table(counts, list(range(lo, lo + len(counts))))
            w, st, nb = rans_encode(col, tab)
            ch.word_offsets.append(sum(len(a) for a in all_words))
            all_words.append(w)
            ch.streams.append(Stream(c, i, len(col), tab, w, st, nb))
    ch.bitstream = np.concatenate(all_words) if all_words else np.zeros(1, np.uint32)
    return ch


def decompress_chunk(ch: Chunk, out_dtype=np.float16) -> np.ndarray:
    """CompressedKVCache._decompress_chunk (llm/compressed_kv_cache.py:289-332):
    decode streams, scatter columns by coset, symbols_to_e8, times the fp16 scale
    (with a dither seed: the dither is subtracted first, fp32 arithmetic)."""
    n = ch.n_vectors
    cos = unpack_coset_bits(ch.coset_packed, n).astype(np.int64)
    syms = np.zeros((n, 8), dtype=np.int64)
    for s in ch.streams:
        rows = np.where(cos == s.coset)[0]
        syms[rows, s.idx] = rans_decode(s.words, s.n_bits, s.state, s.table, s.n_symbols)
    if ch.esc_k is not None:
        for j, words in ch.fine.items():
            k = int(ch.esc_k[j])
            syms[:, j] = (syms[:, j] << k) + unpack_fine(words, k, n)
    q = symbols_to_e8(cos, syms[:, :7], syms[:, 7])
    if ch.dither_seed is not None:
        q = (q - dither(ch.dither_seed, n)).astype(np.float32)
    nh = ch.scales.shape[0]
    sc = ch.scales.astype(np.float32)
    out = (q.reshape(nh, -1, 8) * sc[:, None, None]).astype(np.float32)
    return out.reshape(ch.shape).astype(out_dtype)


def dequant_compact(packed: np.ndarray, bits: int, scales: np.ndarray, head_idx: np.ndarray) -> np.ndarray:
    """triton_unpack_e8_4bit semantics (core/triton_dequant.py:61-132) with the
    floor-mod parity of unpack_e8: fp16((coord + 0.5*coset) * scale[head])."""
    q = unpack_e8(packed, bits)
    s = np.asarray(scales, np.float32)[np.asarray(head_idx)]
    return (q * s[:, None]).astype(np.float32).astype(np.float16)


# ------------------------------------------------------------------ RHT ---

def rht_signs(d: int, seed: int) -> np.ndarray:
    """core/pipeline.py:89-98: signs = where(rand(d, Generator(seed)) < 0.5, +1, -1)."""
    import torch
    g = torch.Generator()
    g.manual_seed(int(seed))
    r = torch.rand(d, generator=g)
    return np.where(r.numpy() < 0.5, 1.0, -1.0).astype(np.float32)


def head_rht_seed(layer_idx: int, head_idx: int, kv_type: int) -> int:
    """llm/perplexity_eval.py:41"""
    return layer_idx * 10000 + head_idx * 10 + kv_type


def fwht(x: np.ndarray) -> np.ndarray:
    """core/pipeline.py:49-69: H x / sqrt(d), float64 reference."""
    y = np.array(x, dtype=np.float64)
    d = y.shape[-1]
    h = 1
    while h < d:
        y = y.reshape(*y.shape[:-1], d // (2 * h), 2, h)
        a = y[..., 0, :].copy()
        b = y[..., 1, :].copy()
        y[..., 0, :] = a + b
        y[..., 1, :] = a - b
        y = y.reshape(*y.shape[:-3], d)
        h *= 2
    return y / np.sqrt(d)


def rht_f32(x: np.ndarray, signs: np.ndarray, inverse: bool = False) -> np.ndarray:
    """RHT.forward / RHT.inverse in float32 (core/pipeline.py:49-69, 100-118):
    butterflies h = 1, 2, .. with (a, b) -> (a + b, a - b), one IEEE division
    by f32(sqrt(d)), signs applied before (forward) or after (inverse)."""
    y = np.array(x, dtype=np.float32, copy=True)
    sg = np.asarray(signs, dtype=np.float32)
    d = y.shape[-1]
    if not inverse:
        y = (y * sg).astype(np.float32)
    h = 1
    while h < d:
        y = y.reshape(*y.shape[:-1], d // (2 * h), 2, h)
        a = y[..., 0, :].copy()
        b = y[..., 1, :].copy()
        y[..., 0, :] = a + b
        y[..., 1, :] = a - b
        y = y.reshape(*y.shape[:-3], d)
        h *= 2
    y = (y / np.float32(np.sqrt(d))).astype(np.float32)
    if inverse:
        y = (y * sg).astype(np.float32)
    return y


# ------------------------------------------------------------ attention ---

def decode_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """softmax(q K^T / sqrt(hd)) V in float64 with GQA (q head h reads kv head h // group).
    q: (B, Hq, 1, hd); k, v: (B, Hkv, S, hd) -> (B, Hq, 1, hd)"""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Hq, _, hd = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    out = np.empty((B, Hq, 1, hd))
    for b in range(B):
        for h in range(Hq):
            kh = k[b, h // g]
            s = kh @ q[b, h, 0] / math.sqrt(hd)
            s = np.exp(s - s.max())
            out[b, h, 0] = (s[:, None] * v[b, h // g]).sum(0) / s.sum()
    return out
