"""Bit-wise streaming rANS on gfx950 (API of reference core/gpu_ans.py).

Format (core/gpu_ans.py:44-139): precision L = 1024 (LOG2_L = 10), state in
[L, 2L), one renormalisation bit at a time.  The encoder walks the symbols in
reverse; the emitted bit list is reversed and packed LSB-first into uint32
words, followed by one zero word.  Tables are normalised to sum L with the
reference's adjustment loop, including numpy's argsort tie order.

Every function here runs its arithmetic in liblatticequant_amd.so:
build_rans_table -> lq_build_tables, rans_encode -> lq_symbol_index +
lq_rans_encode_streams, rans_decode_cpu / the GPU decoder ->
lq_rans_decode_streams.  Host numpy arrays are accepted and returned where the
reference takes and returns them; a GPU is required.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import numpy as np
import torch

from .. import _lib as L_

LOG2_L = 10
L = 1 << LOG2_L  # 1024


def _dev(device=None) -> torch.device:
    L_.lib()
    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    d = torch.device(device)
    if d.type != "cuda":
        raise ValueError(f"the rANS kernels run on a ROCm device, not {d}")
    return d if d.index is not None else torch.device("cuda", torch.cuda.current_device())


@dataclass
class RANSTable:
    """Precomputed rANS table (core/gpu_ans.py:52-59)."""
    lookup: np.ndarray      # (L,) int32 -- slot -> symbol index
    freqs: np.ndarray       # (n_symbols,) int32
    cumfreqs: np.ndarray    # (n_symbols + 1,) int32
    alphabet: List[int]
    n_symbols: int
    # device status bits of the table build (0: the table equals build_rans_table's,
    # numpy's argsort tie order included)
    status: int = 0


def build_rans_tables(counts_list, alphabets, device=None) -> List[RANSTable]:
    """Several tables in one launch (one workgroup each).  See build_rans_table."""
    dev = _dev(device)
    n_t = len(counts_list)
    if n_t == 0:
        return []
    sizes = [len(a) for a in alphabets]
    for c, n in zip(counts_list, sizes):
        if len(c) != n:
            raise ValueError("counts and alphabet lengths differ")
        if n > L:
            raise ValueError(f"alphabet of {n} symbols exceeds L={L}: the reference's "
                             "normalisation loop never terminates there")
        if n == 0:
            raise ValueError("empty alphabet")
    off = np.zeros(n_t + 1, np.int64)
    off[1:] = np.cumsum(sizes)
    flat = np.concatenate([np.asarray(c).astype(np.int64, copy=False).reshape(-1) for c in counts_list])
    d_counts = torch.from_numpy(flat).to(dev)
    d_off = torch.from_numpy(off[:-1].copy()).to(dev)
    d_n = torch.tensor(sizes, dtype=torch.int32, device=dev)
    d_freqs = torch.empty(int(off[-1]), dtype=torch.int32, device=dev)
    d_cum = torch.empty(int(off[-1]) + n_t, dtype=torch.int32, device=dev)
    d_lookup = torch.empty(n_t * L, dtype=torch.int32, device=dev)
    d_st = torch.empty(n_t, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        L_.check(L_.lib().lq_build_tables(d_counts.data_ptr(), d_off.data_ptr(), d_n.data_ptr(), n_t,
                                          d_freqs.data_ptr(), d_cum.data_ptr(), d_lookup.data_ptr(),
                                          d_st.data_ptr(), L_.stream_ptr(dev)), "lq_build_tables")
    freqs = d_freqs.cpu().numpy()
    cum = d_cum.cpu().numpy()
    lookup = d_lookup.cpu().numpy().reshape(n_t, L)
    st = d_st.cpu().numpy()
    out = []
    for t in range(n_t):
        if st[t] & L_.LQ_ST_ALPHABET:
            raise ValueError("alphabet exceeds L")
        a, b = int(off[t]), int(off[t + 1])
        out.append(RANSTable(lookup=lookup[t].copy(), freqs=freqs[a:b].copy(), cumfreqs=cum[a + t:b + t + 1].copy(),
                             alphabet=list(alphabets[t]), n_symbols=sizes[t], status=int(st[t])))
    return out


def build_rans_table(counts: np.ndarray, alphabet: List[int]) -> RANSTable:
    """Normalise counts to sum L, then cumfreqs and the slot -> symbol lookup.
    core/gpu_ans.py:62-98.  An alphabet above L raises ValueError (the
    reference's loop does not terminate there)."""
    return build_rans_tables([counts], [list(alphabet)])[0]


def _contiguous(alphabet) -> bool:
    a = np.asarray(alphabet, dtype=np.int64)
    return len(a) > 0 and bool(np.all(np.diff(a) == 1))


def _encode_many(symbol_lists, tables, dev):
    """Encode several streams in one launch (one lane per stream)."""
    lib = L_.lib()
    s = L_.stream_ptr(dev)
    n_s = len(symbol_lists)
    lens = np.array([len(x) for x in symbol_lists], np.int64)
    sym_off = np.zeros(n_s, np.int64)
    sym_off[1:] = np.cumsum(lens)[:-1]
    idx = torch.empty(max(int(lens.sum()), 1), dtype=torch.int32, device=dev)
    # symbol -> index, per stream (its own alphabet)
    for i, (syms, tab) in enumerate(zip(symbol_lists, tables)):
        if lens[i] == 0:
            continue
        d_sym = torch.as_tensor(np.asarray(syms).astype(np.int64, copy=False)).to(dev)
        d_alph = torch.tensor(list(tab.alphabet), dtype=torch.int64, device=dev)
        o = int(sym_off[i])
        L_.check(lib.lq_symbol_index(d_sym.data_ptr(), int(lens[i]), d_alph.data_ptr(), tab.n_symbols,
                                     1 if _contiguous(tab.alphabet) else 0, idx[o:].data_ptr(), s), "lq_symbol_index")
    tab_sizes = np.array([t.n_symbols for t in tables], np.int64)
    tab_off = np.zeros(n_s, np.int64)
    tab_off[1:] = np.cumsum(tab_sizes + 1)[:-1]
    freqs = np.zeros(int((tab_sizes + 1).sum()), np.int32)
    cum = np.zeros_like(freqs)
    for i, t in enumerate(tables):
        o = int(tab_off[i])
        freqs[o:o + t.n_symbols] = t.freqs
        cum[o:o + t.n_symbols + 1] = t.cumfreqs
    cap = (10 * lens + 31) // 32 + 2
    word_off = np.zeros(n_s, np.int64)
    word_off[1:] = np.cumsum(cap)[:-1]
    tw = int(cap.sum())
    d_words = torch.empty(tw, dtype=torch.int32, device=dev)
    d_scr = torch.empty(tw, dtype=torch.int32, device=dev)
    d_state = torch.empty(n_s, dtype=torch.int64, device=dev)
    d_nbits = torch.empty(n_s, dtype=torch.int64, device=dev)
    tt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    d_sym_off, d_lens, d_tab_off, d_word_off = tt(sym_off), tt(lens), tt(tab_off), tt(word_off)
    d_freqs, d_cum = tt(freqs), tt(cum)
    L_.check(lib.lq_rans_encode_streams(idx.data_ptr(), d_sym_off.data_ptr(), d_lens.data_ptr(), d_freqs.data_ptr(),
                                        d_cum.data_ptr(), d_tab_off.data_ptr(), n_s, d_scr.data_ptr(),
                                        d_words.data_ptr(), d_word_off.data_ptr(), d_state.data_ptr(),
                                        d_nbits.data_ptr(), s), "lq_rans_encode_streams")
    words = d_words.cpu().numpy().view(np.uint32)
    state = d_state.cpu().numpy()
    nbits = d_nbits.cpu().numpy()
    out = []
    for i in range(n_s):
        nw = (int(nbits[i]) + 31) // 32
        o = int(word_off[i])
        out.append((words[o:o + nw + 1].copy(), int(state[i]), int(nbits[i])))
    return out


def rans_encode_many(symbol_lists, tables, device=None) -> List[Tuple[np.ndarray, int, int]]:
    """rans_encode over several (symbols, table) pairs in one kernel launch."""
    dev = _dev(device)
    with torch.cuda.device(dev):
        return _encode_many(symbol_lists, tables, dev)


def rans_encode(symbols: np.ndarray, table: RANSTable) -> Tuple[np.ndarray, int, int]:
    """Streaming rANS encode (reverse order).  core/gpu_ans.py:105-139
    Returns (bitstream uint32 [n_words + 1], initial state for decode, n_bits).
    A symbol outside the alphabet encodes as its nearest alphabet entry."""
    return rans_encode_many([symbols], [table])[0]


def rans_decode_cpu(bitstream: np.ndarray, n_bits: int, state: int, table: RANSTable,
                    n_symbols: int) -> np.ndarray:
    """Decode one stream (core/gpu_ans.py:146-168).  The name is the
    reference's; the decode runs in the lq_rans_decode_streams kernel."""
    st = RANSStream(bitstream=np.asarray(bitstream), n_bits=int(n_bits), initial_state=int(state),
                    n_symbols=int(n_symbols), table=table)
    return gpu_rans_decode([st])[0]


@dataclass
class RANSStream:
    """One encoded stream ready for GPU decode (core/gpu_ans.py:242-248)."""
    bitstream: np.ndarray
    n_bits: int
    initial_state: int
    n_symbols: int
    table: RANSTable


@dataclass
class PreparedGPUDecode:
    """Device tensors of a batch of streams (core/gpu_ans.py:252-271)."""
    d_bits: torch.Tensor
    d_bit_off: torch.Tensor
    d_nbits: torch.Tensor
    d_init: torch.Tensor
    d_ndec: torch.Tensor
    d_lookup: torch.Tensor
    d_freqs: torch.Tensor
    d_cumfreqs: torch.Tensor
    d_alphabet: torch.Tensor
    d_tid: torch.Tensor
    d_out: torch.Tensor
    d_out_off: torch.Tensor
    max_sym: int
    max_decode: int
    n_streams: int
    out_offsets: List[int]
    stream_lengths: List[int]


def prepare_gpu_decode(streams: List[RANSStream], device: str = "cuda") -> PreparedGPUDecode:
    """Flatten the streams' bitstreams and (deduplicated) tables into device
    tensors with the reference's layout (core/gpu_ans.py:274-342)."""
    dev = _dev(device)
    n_streams = len(streams)
    max_sym = max(s.table.n_symbols for s in streams)
    max_decode = max(s.n_symbols for s in streams)
    bit_offsets, total = [], 0
    words = []
    for s in streams:
        bit_offsets.append(total)
        w = np.asarray(s.bitstream)
        words.append(w.view(np.int32) if w.dtype in (np.uint32, np.int32) else w.astype(np.uint32).view(np.int32))
        total += len(w) * 32
    flat = np.concatenate(words) if words else np.zeros(1, np.int32)
    tmap, tlist, tids = {}, [], []
    for s in streams:
        k = id(s.table)
        if k not in tmap:
            tmap[k] = len(tlist)
            tlist.append(s.table)
        tids.append(tmap[k])
    nt = len(tlist)
    lookup = np.zeros((nt, L), np.int32)
    freqs = np.zeros((nt, max_sym), np.int32)
    cum = np.zeros((nt, max_sym), np.int32)
    alph = np.zeros((nt, max_sym), np.int32)
    for i, t in enumerate(tlist):
        lookup[i] = t.lookup
        freqs[i, :t.n_symbols] = t.freqs
        cum[i, :t.n_symbols] = t.cumfreqs[:t.n_symbols]
        alph[i, :t.n_symbols] = np.asarray(t.alphabet, np.int64).astype(np.int32)
    out_off, tot_out, lens = [], 0, []
    for s in streams:
        out_off.append(tot_out)
        tot_out += s.n_symbols
        lens.append(s.n_symbols)
    i32 = lambda a: torch.tensor(np.asarray(a, dtype=np.int32).reshape(-1), dtype=torch.int32, device=dev)  # noqa: E731
    return PreparedGPUDecode(
        d_bits=torch.from_numpy(np.ascontiguousarray(flat)).to(dev), d_bit_off=i32(bit_offsets),
        d_nbits=i32([s.n_bits for s in streams]), d_init=i32([s.initial_state for s in streams]),
        d_ndec=i32([s.n_symbols for s in streams]), d_lookup=i32(lookup), d_freqs=i32(freqs),
        d_cumfreqs=i32(cum), d_alphabet=i32(alph), d_tid=i32(tids),
        d_out=torch.zeros(max(tot_out, 1), dtype=torch.int64, device=dev), d_out_off=i32(out_off),
        max_sym=max_sym, max_decode=max_decode, n_streams=n_streams, out_offsets=out_off, stream_lengths=lens)


def run_gpu_decode_kernel(prep: PreparedGPUDecode):
    """Decode every stream, one lane each (core/gpu_ans.py:345-354)."""
    dev = prep.d_out.device
    with torch.cuda.device(dev):
        prep.d_out.zero_()
        L_.check(L_.lib().lq_rans_decode_streams(
            prep.d_bits.data_ptr(), prep.d_bit_off.data_ptr(), prep.d_nbits.data_ptr(), prep.d_init.data_ptr(),
            prep.d_ndec.data_ptr(), prep.d_lookup.data_ptr(), prep.d_freqs.data_ptr(), prep.d_cumfreqs.data_ptr(),
            prep.d_alphabet.data_ptr(), prep.d_tid.data_ptr(), prep.max_sym, prep.d_out_off.data_ptr(),
            prep.n_streams, prep.d_out.data_ptr(), L_.stream_ptr(dev)), "lq_rans_decode_streams")


def extract_gpu_results(prep: PreparedGPUDecode) -> List[np.ndarray]:
    """Copy back and split by stream (core/gpu_ans.py:357-361)."""
    out = prep.d_out.cpu().numpy()
    return [out[prep.out_offsets[i]:prep.out_offsets[i] + prep.stream_lengths[i]] for i in range(prep.n_streams)]


def gpu_rans_decode(streams: List[RANSStream], device: str = "cuda") -> List[np.ndarray]:
    """prepare + kernel + extract (core/gpu_ans.py:364-370)."""
    if not streams:
        return []
    prep = prepare_gpu_decode(streams, device)
    run_gpu_decode_kernel(prep)
    return extract_gpu_results(prep)
