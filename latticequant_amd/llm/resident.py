"""Resident (fixed-width) form of a compressed KV prefix and decode attention over it.

The rANS chunks of :mod:`latticequant_amd.codec` are the cache's at-rest form,
bit-exact with the reference's bitstreams.  A decode step needs the prefix at
every step, and re-running rANS over 32k tokens per step is instruction-bound,
so the cache also keeps the same lattice points as one b = 5 fixed-rate code
word per vector (the ``pack_e8`` word of core/compact_storage.py:87-154,
split into a 32-bit and an 8-bit plane laid out for the attention kernel's
MFMA operands), with an exception entry (the lattice point as int16 2c) for
every vector outside the 5-bit range -- the representable / fallback split of
llm/fused_triton_merge.py:33-130.  At 4 bits/dim a prefix costs about 5.3 B
per 8-dim vector here, against 16 B for the fp16 cache the reference keeps
resident beside its chunks (llm/compressed_kv_cache.py:384-395).

``resident_decode_attention`` is one decode step of
softmax(q K^T / sqrt(128)) V over a resident K / V prefix plus an fp16 tail
(lq_resident_attention: MFMA for Q K^T and P V, online softmax, split-token
records merged in the same launch).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from .. import _lib as L

RB = 16          # tokens per resident block
HD = 128


class ResidentKV:
    """Resident prefix of n_heads kv heads (B * H_kv), capacity cap_tokens tokens each."""

    def __init__(self, n_heads: int, cap_tokens: int, device=None, exc_cap: Optional[int] = None):
        if n_heads <= 0 or cap_tokens <= 0:
            raise ValueError("n_heads and cap_tokens must be positive")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        nb = (cap_tokens + RB - 1) // RB
        self.device = dev
        self.n_heads = int(n_heads)
        self.cap_blocks = nb
        self.a = torch.zeros(n_heads * nb * 64 * 4, dtype=torch.int32, device=dev)
        self.b = torch.zeros(n_heads * nb * 64 * 4, dtype=torch.uint8, device=dev)
        self.mask = torch.zeros(n_heads * nb * 4, dtype=torch.int64, device=dev)
        self.meta = torch.zeros(n_heads * nb * 4, dtype=torch.int32, device=dev)
        self.scale = torch.zeros(n_heads * nb * RB, dtype=torch.float16, device=dev)
        self.n_exc = torch.zeros(1, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        cap = exc_cap if exc_cap is not None else max(256, n_heads * nb * 4)
        self.exc = torch.zeros(cap * 8, dtype=torch.int16, device=dev)
        self.n_tokens = 0
        # exception count as the host knows it without waiting: a count read
        # back earlier (pinned copy + event), the vectors appended after it
        # (each may add one exception), and the newest read still in flight
        self._exc_known = 0
        self._exc_since = 0
        self._exc_read = None   # (pinned count, event, vectors appended after its snapshot)
        self._st = None         # the ctypes view of the buffers, rebuilt when one is reallocated

    @property
    def exc_cap(self) -> int:
        return self.exc.numel() // 8

    def struct(self) -> L.Resident:
        """The buffers as the C ABI's lq_resident (cached: the pointers and
        capacities change only when reserve() or the exception list grows)."""
        if self._st is None:
            self._st = L.Resident(a=self.a.data_ptr(), b=self.b.data_ptr(), mask=self.mask.data_ptr(),
                                  meta=self.meta.data_ptr(), exc=self.exc.data_ptr(), scale=self.scale.data_ptr(),
                                  n_exc=self.n_exc.data_ptr(), status=self.status.data_ptr(), n_heads=self.n_heads,
                                  cap_blocks=self.cap_blocks, exc_cap=self.exc_cap)
        return self._st

    def nbytes(self) -> int:
        """Bytes a decode step reads per token range: records, masks, bases, scales, exceptions in use."""
        nb = (self.n_tokens + RB - 1) // RB
        per_blk = 64 * 4 * 4 + 64 * 4 + 16 + RB * 2   # records, meta, scales
        return self.n_heads * nb * per_blk + int(self.n_exc.item()) * 16

    def reserve(self, cap_tokens: int) -> None:
        """Grow the capacity to at least cap_tokens tokens per head (copies the blocks in use)."""
        nb = (cap_tokens + RB - 1) // RB
        if nb <= self.cap_blocks:
            return
        H, ob = self.n_heads, self.cap_blocks
        used = (self.n_tokens + RB - 1) // RB

        def grow(t, per_blk):
            n = torch.zeros(H * nb * per_blk, dtype=t.dtype, device=t.device)
            n.view(H, nb, per_blk)[:, :used].copy_(t.view(H, ob, per_blk)[:, :used])
            return n
        self.a = grow(self.a, 64 * 4)
        self.b = grow(self.b, 64 * 4)
        self.mask = grow(self.mask, 4)
        self.meta = grow(self.meta, 4)
        self.scale = grow(self.scale, RB)
        self.cap_blocks = nb
        self._st = None

    # appends of at most this many vectors run without a host read: the
    # exception list is grown (device copy) whenever the host's upper bound of
    # the count could pass its capacity; larger appends (a prefill) read the
    # count back instead, so that the list does not grow to the bound
    ASYNC_MAX_VECTORS = 1 << 14

    def append(self, x: torch.Tensor, scale32: torch.Tensor, scale16: torch.Tensor) -> None:
        """Quantize x (B, H, T, 128) with the per-head scales of its chunk
        (B*H of each; the points are those the chunk codec codes with the same
        scale32) and append it: T must be a multiple of 16.  Small appends (a
        decode step's flush) make no host read; larger ones grow the exception
        list to its exact need (one or two host reads of the count)."""
        if x.dim() != 4 or x.shape[3] != HD:
            raise ValueError("x must be (B, H, T, 128)")
        B, H, T, _ = x.shape
        if B * H != self.n_heads:
            raise ValueError(f"x has {B * H} heads, the resident prefix {self.n_heads}")
        if T % RB:
            raise ValueError(f"resident blocks hold {RB} tokens: append a multiple of {RB} (keep the rest in the tail)")
        if self.n_tokens % RB:
            raise ValueError("resident prefix ends inside a block")
        if self.n_tokens + T > self.cap_blocks * RB:
            raise ValueError("resident prefix capacity exceeded")
        lib = L.lib()
        xc = x.to(self.device).contiguous()
        s32 = scale32.to(device=self.device, dtype=torch.float32).contiguous().view(-1)
        s16 = scale16.to(device=self.device, dtype=torch.float16).contiguous().view(-1)
        if s32.numel() != self.n_heads or s16.numel() != self.n_heads:
            raise ValueError("one scale per head expected")
        work = torch.empty(int(lib.lq_resident_workspace(self.n_heads, T)), dtype=torch.uint8, device=self.device)
        blk0 = self.n_tokens // RB
        n_new = self.n_heads * T * (HD // 8)   # vectors appended: each can be one exception

        def launch():
            st = self.struct()
            L.check(lib.lq_resident_quantize(xc.data_ptr(), L.dtype_code(xc.dtype), self.n_heads, T,
                                             s32.data_ptr(), s16.data_ptr(), ctypes.addressof(st), 0, blk0,
                                             work.data_ptr(), L.stream_ptr(self.device)), "lq_resident_quantize")

        with torch.cuda.device(self.device):
            if n_new <= self.ASYNC_MAX_VECTORS:
                if self._exc_read is not None and self._exc_read[1].query():
                    host, _, after = self._exc_read
                    self._exc_known, self._exc_since, self._exc_read = int(host[0]), after, None
                need = self._exc_known + self._exc_since + n_new
                if need > self.exc_cap:
                    self._grow_exc(max(2 * self.exc_cap, need), self.exc_cap)
                launch()
                self._exc_since += n_new
                if self._exc_read is not None:
                    host, ev, after = self._exc_read
                    self._exc_read = (host, ev, after + n_new)
                else:
                    host = torch.empty(1, dtype=torch.int32, pin_memory=True)
                    host.copy_(self.n_exc, non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(torch.cuda.current_stream(self.device))
                    self._exc_read = (host, ev, 0)
            else:
                n0 = int(self.n_exc.item())
                for attempt in range(2):
                    launch()
                    n1 = int(self.n_exc.item())
                    if n1 <= self.exc_cap:
                        break
                    # grow the exception list to the exact need and redo this append
                    self._grow_exc(max(n1, 2 * self.exc_cap), n0)
                    self.n_exc.fill_(n0)
                    self.status.zero_()
                self._exc_known, self._exc_since, self._exc_read = n1, 0, None
        self.n_tokens += T

    def _grow_exc(self, cap: int, keep: int) -> None:
        """A longer exception list holding the first `keep` entries."""
        grown = torch.zeros(cap * 8, dtype=torch.int16, device=self.device)
        grown[:keep * 8] = self.exc[:keep * 8]
        self.exc = grown
        self._st = None

    def dequant(self, out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """(n_heads, n_tokens, 128): lattice point times the stored fp16 scale,
        rounded once (the values _decompress_chunk writes)."""
        lib = L.lib()
        nb = self.n_tokens // RB
        out = torch.empty(self.n_heads, nb * RB, HD, dtype=out_dtype, device=self.device)
        if nb:
            st = self.struct()
            with torch.cuda.device(self.device):
                L.check(lib.lq_resident_dequant(ctypes.addressof(st), 0, self.n_heads, 0, nb, out.data_ptr(),
                                                L.dtype_code(out_dtype), L.stream_ptr(self.device)),
                        "lq_resident_dequant")
        return out


def from_chunk(x: torch.Tensor, enc, cap_tokens: Optional[int] = None) -> ResidentKV:
    """Resident form of one chunk (x (B, H, T, 128) and its EncodedBatch enc of
    one chunk): the same lattice points as enc's bitstreams."""
    B, H, T, _ = x.shape
    r = ResidentKV(B * H, cap_tokens or T, device=x.device)
    r.append(x, enc.scale32.view(-1)[:B * H], enc.scale16.view(-1)[:B * H])
    return r


def attn_workspace(n_heads: int, group: int, t_prefix: int, t_tail: int, device=None) -> torch.Tensor:
    """Workspace of lq_resident_attention (counters zeroed; each call leaves them zero)."""
    n = L.lib().lq_resident_attn_workspace(n_heads, group, t_prefix, t_tail)
    if n < 0:
        raise ValueError("bad attention geometry")
    return torch.zeros(int(n), dtype=torch.uint8, device=device)


def resident_decode_attention(k: ResidentKV, v: ResidentKV, q: torch.Tensor, tail_k: Optional[torch.Tensor] = None,
                              tail_v: Optional[torch.Tensor] = None, work: Optional[torch.Tensor] = None,
                              out: Optional[torch.Tensor] = None, t_prefix: Optional[int] = None) -> torch.Tensor:
    """q: (B, Hq, 1, 128) fp16, Hq = group * H_kv (group 1..16); k / v: resident
    prefixes of B * H_kv heads; tail_k / tail_v: (B, H_kv, Tt, 128) fp16 or None.
    Returns (B, Hq, 1, 128) fp16 = softmax(q K^T / sqrt(128)) V over prefix + tail."""
    lib = L.lib()
    if k.n_heads != v.n_heads or k.n_tokens != v.n_tokens:
        raise ValueError("K and V resident prefixes must have the same geometry")
    tp = k.n_tokens if t_prefix is None else int(t_prefix)
    if tp < 0 or tp > k.n_tokens or tp % RB:
        raise ValueError("t_prefix must be a multiple of 16 within the resident prefix")
    if q.dtype != torch.float16 or q.dim() != 4 or q.shape[2] != 1 or q.shape[3] != HD:
        raise ValueError("q must be (B, Hq, 1, 128) fp16")
    B, Hq = q.shape[0], q.shape[1]
    if B < 1 or k.n_heads % B:
        raise ValueError("the resident prefix must hold B * H_kv heads")
    Hkv = k.n_heads // B
    if Hq % Hkv:
        raise ValueError("query heads must be a multiple of the kv heads")
    group = Hq // Hkv
    if not 1 <= group <= 16:
        raise ValueError("group (query heads per kv head) must be 1..16")
    dev = k.device
    tt = 0
    pk = pv = None
    if tail_k is not None and tail_k.shape[2] > 0:
        if tail_v is None or tail_k.shape != tail_v.shape or tail_k.shape[:2] != (B, Hkv) or tail_k.shape[3] != HD:
            raise ValueError("tail K / V must be (B, H_kv, Tt, 128)")
        tt = int(tail_k.shape[2])
        pk = tail_k.to(device=dev, dtype=torch.float16).contiguous()
        pv = tail_v.to(device=dev, dtype=torch.float16).contiguous()
    if tp + tt == 0:
        raise ValueError("empty prefix and tail")
    need = lib.lq_resident_attn_workspace(k.n_heads, group, tp, tt)
    if work is None:
        work = attn_workspace(k.n_heads, group, tp, tt, dev)
    elif work.numel() < need:
        raise ValueError("attention workspace too small")
    qc = q.to(dev).contiguous()
    if out is None:
        out = torch.empty(B, Hq, 1, HD, dtype=torch.float16, device=dev)
    ks, vs = k.struct(), v.struct()

    def call():
        L.check(lib.lq_resident_attention(ctypes.addressof(ks), ctypes.addressof(vs), tp, qc.data_ptr(), group,
                                          L.ptr(pk), L.ptr(pv), tt, work.data_ptr(), out.data_ptr(),
                                          L.stream_ptr(dev)), "lq_resident_attention")
    if dev.index == torch.cuda.current_device():
        call()
    else:
        with torch.cuda.device(dev):
            call()
    return out
