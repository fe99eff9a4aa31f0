"""Benchmark of the E8 + rANS compressed-KV hot path on one MI355X.

Headline workload ("C2"): a Llama-3.1-8B-shaped KV
cache, 32 layers x {K, V} x [batch 1, 8 kv heads, 8192 tokens, head_dim 128]
fp16, N(0, 1) with 4 fixed outlier channels per head scaled x10, 4 bits/dim,
one chunk (one _compress_tensor call, per-chunk tables) per layer and K/V.
Inputs come from torch's CPU generator (seed 1000*layer + kv), their SHA-256
is in the line, and they are resident in HBM before timing starts.

One step = write (compress all 64 chunks: scales, E8, tables, rANS encode,
bitstream assembly) + read (decode + dequantise all 64 chunks back to fp16).

value = algorithmic bytes / time with B = 4*D + 2*C (write reads 2D fp16
bytes and writes C; read reads C and writes 2D), D = fp16 elements,
C = stored compressed bytes (bitstream + coset bits + scales + tables +
checkpoints).

Also on the line, each with its own roofline fraction: C3 (the 32k-context
decode step), C1 (fixed-rate round trip), C4 (28-layer 3/4/5-bit schedule,
heavy-tailed K) and C5 (batch-8 x 131072-token rotated + dithered cache,
sustained write and read); and cpu_baseline with three CPU tiers (oracle on one
core, oracle on every affinity core, the reference's as-written structure on a
slice), the core count, torch's threads and the CPU model.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
                    [--skip c1,c3,c4,c5] [--c5-layers N]
    python bench.py --only c1|c3|c4|c5      one leg alone (the profiling entry points)
    python bench.py --e2e                   model decode tok/s through the HF cache interface
"""
import argparse
import dataclasses
import hashlib
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "E8+rANS KV GB/s (write+read) and 32k-ctx compressed decode step µs, 1 GPU"
HBM_PEAK_GBS = 8000.0

LAYERS, HEADS, TOKENS, HD, BITS = 32, 8, 8192, 128, 4


def _sha(t: torch.Tensor) -> str:
    """SHA-256 of a CPU tensor's bytes."""
    return hashlib.sha256(memoryview(t.contiguous().numpy()).cast("B")).hexdigest()


def make_kv(device):
    """C2 input: 64 chunks (layer-major, K then V), each N(0,1) from torch's CPU
    generator seeded 1000*layer + kv, 4 outlier channels per head
    (randperm(128)[:4] of a second CPU generator with the same seed, one draw
    per head) scaled x10, rounded to fp16, moved to `device`.
    Returns (x, SHA-256 over the fp16 bytes of the 64 chunks in order)."""
    x = torch.empty(LAYERS * 2, 1, HEADS, TOKENS, HD, dtype=torch.float16, device=device)
    h = hashlib.sha256()
    for layer in range(LAYERS):
        for kv in range(2):
            t = torch.randn(HEADS, TOKENS, HD, generator=torch.Generator().manual_seed(1000 * layer + kv))
            gc = torch.Generator().manual_seed(1000 * layer + kv)
            for hd_ in range(HEADS):
                ch = torch.randperm(HD, generator=gc)[:4]
                t[hd_][:, ch] *= 10.0
            t16 = t.to(torch.float16)
            h.update(memoryview(t16.numpy()).cast("B"))
            x[2 * layer + kv, 0] = t16.to(device)
    return x, h.hexdigest()


def cpu_info():
    """Cores this process may use, torch's intra-op threads and the CPU model."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"affinity_cores": len(os.sched_getaffinity(0)), "torch_threads": torch.get_num_threads(),
            "cpu_model": model}


def _port_chunk(args):
    """One C2 chunk through the oracle (compress + decompress) in a worker
    process; returns its algorithmic bytes 4 D + 2 C."""
    t, sc, bits = args
    from oracle import oracle as O
    ch = O.compress_chunk(t, bits, scales_f32=sc)
    O.decompress_chunk(ch)
    return 4 * t.size + 2 * ch.compressed_bytes


def _port_ready(_):
    from oracle import oracle as O
    O.lib()
    return os.getpid()


def cpu_baseline(x_chunks, bits, scale_rows, gpu_words, gpu_out):
    """CPU baselines of C2 on the GPU box's host, bounded samples, byte formula
    B = 4 D + 2 C as on the GPU:
      port        the C/numpy oracle, one thread, on len(x_chunks) chunks, each
                  checked bit for bit against the GPU's stream words and decoded
                  output of the same chunk;
      port_cores  the same oracle in one worker process per affinity core (one
                  chunk each; processes, since the numpy parts hold the GIL);
      as_written  the reference's CPU structure (oracle/aswritten.py: torch-CPU
                  E8 on all torch threads, per-symbol Python rANS loops on one)
                  on 1/64 of one chunk (128 of its 8192 tokens), extrapolated
                  linearly to the full cache.
    Returns (tiers, indices of the bit-exact chunks)."""
    import multiprocessing as mp
    from concurrent.futures import ProcessPoolExecutor
    from oracle import aswritten as A
    from oracle import oracle as O
    info = cpu_info()
    tiers = {}
    t0 = time.perf_counter()
    nbytes, exact = 0, []
    for i, (t, sc) in enumerate(zip(x_chunks, scale_rows)):
        ch = O.compress_chunk(t, bits, scales_f32=sc)
        dec = O.decompress_chunk(ch)
        nbytes += 4 * t.size + 2 * ch.compressed_bytes
        if np.array_equal(gpu_words[i], ch.bitstream) and np.array_equal(gpu_out[i], dec):
            exact.append(i)
    dt = time.perf_counter() - t0
    tiers["port"] = {"value": round(nbytes / dt / 1e9, 5), "unit": "GB/s", "cores": 1, "kind": "port",
                     "wall_s": round(dt, 2),
                     "sample": f"{len(x_chunks)} of the 64 C2 chunks ([1,8,8192,128] fp16 each): compress + "
                               f"decompress with the single-threaded C/numpy oracle"}
    nc = max(1, info["affinity_cores"])
    jobs = [(x_chunks[i % len(x_chunks)], scale_rows[i % len(x_chunks)], bits) for i in range(nc)]
    with ProcessPoolExecutor(max_workers=nc, mp_context=mp.get_context("spawn")) as ex:
        list(ex.map(_port_ready, range(nc)))          # workers started and the oracle loaded, untimed
        t0 = time.perf_counter()
        nb = sum(ex.map(_port_chunk, jobs))
        dt = time.perf_counter() - t0
    tiers["port_cores"] = {"value": round(nb / dt / 1e9, 5), "unit": "GB/s", "cores": nc, "kind": "port",
                           "wall_s": round(dt, 2),
                           "sample": f"{nc} C2 chunks, one per worker process on {nc} affinity cores"}
    t = x_chunks[0][:, :, :TOKENS // 64]
    t0 = time.perf_counter()
    streams, s16, cos = A.compress(torch.from_numpy(t), bits, scales_f32=scale_rows[0])
    A.decompress(streams, cos, s16, t.shape)
    dt = time.perf_counter() - t0
    csz = sum(len(st[2]) for st in streams) * 4 + (len(cos) + 7) // 8 + 2 * HEADS
    b_slice = 4 * t.size + 2 * csz
    tiers["as_written"] = {"value": round(b_slice / dt / 1e9, 7), "unit": "GB/s",
                           "cores": info["torch_threads"], "kind": "port", "wall_s": round(dt, 2),
                           "extrapolated_full_cache_s": round(dt * 64 * 64, 0),
                           "sample": "1/64 of one C2 chunk ([1,8,128,128] fp16): torch-CPU E8 on "
                                     f"{info['torch_threads']} threads, per-symbol Python rANS table / encode / "
                                     "decode on one, as the reference structures them; the full cache time is "
                                     "that slice x 64 x 64 (extrapolated)"}
    return tiers, exact, info


class CacheFlush:
    """Evicts L2 and MALL before a timed run by reading (summing) a 512 MiB
    buffer: the caches then hold clean lines of unrelated data, the state a
    step meets after other kernels have streamed their inputs.  With
    write=True it writes the buffer instead, which also leaves MALL full of
    dirty lines that the timed kernel must write back as it reads (kept as a
    second, pessimistic measurement)."""

    def __init__(self, dev, write=False, nbytes=512 << 20):
        self.write = write
        self.buf = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
        self.acc = torch.zeros((), dtype=torch.float32, device=dev)

    def __call__(self, i):
        if self.write:
            self.buf.fill_(float(i & 0xff))
        else:
            torch.sum(self.buf, dim=0, out=self.acc)


def timed_median(fn, n, flush=None):
    """Median event time (us) of fn over n runs on the current stream.  Before
    each run: the cache flush (CacheFlush) when given, then a queued GPU spin,
    so the start event is reached after the host has submitted fn."""
    ts = []
    for i in range(n):
        if flush is not None:
            flush(i)
        gpu_busy()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3)
    ts.sort()
    return ts[len(ts) // 2]


def _roof(nbytes, us, what):
    ach = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "bytes": int(nbytes), "us": round(us, 2), "what": what}


def bench_c1(dev, iters=20):
    """C1: K [1,8,2048,128] = randn(fp32, CPU
    generator seed 0).half(), 4 bits/dim, no entropy coding: quantize ->
    fixed-rate compact form (4-byte words of the in-range vectors, fp16
    fallback for the rest, 1-bit mask, per-head scales) -> fused merge back to
    fp16.  B = 4 D + 2 P, P = 4 V_in + 16 V_oor + ceil(V/8) + 2 H.

    Timed: the device round trip (codec.compact_encode: sigma^2 partial sums,
    then one pass that finalises the scales, quantizes, packs and compacts;
    codec.compact_merge: no host sync); the round trip through the API
    (compress_fixed_rate, whose one host sync reads the row counts that size
    the chunk's tensors, then fused_decompress_chunk); and the merge kernel
    alone (the reference's own throughput method,
    core/triton_dequant.py:238-286), with its own look-back over the mask and
    with the encoder's tile offsets; each after a 512 MiB cache flush and warm
    (the 12 MB working set then sits in the 256 MB MALL)."""
    from latticequant_amd import codec
    from latticequant_amd.llm.compressed_kv_cache import compress_fixed_rate
    from latticequant_amd.llm.fused_triton_merge import fused_decompress_chunk
    from oracle import oracle as O
    k = torch.randn(1, 8, 2048, 128, generator=torch.Generator().manual_seed(0)).half()
    sha = _sha(k)
    kd = k.to(dev)
    ch = compress_fixed_rate(kd, 4)
    out = fused_decompress_chunk(ch)
    # parity: lattice points (at the fp32 scales the device quantized with), mask,
    # packed words and merged fp16 (at the stored fp16 scales) against the oracle
    s32 = codec.quantize_points(kd, 4)[1].cpu().numpy()
    qo = O.quantize_heads(k.float().numpy(), s32)
    mask = O.check_representable(qo, 4)
    sw = ch.scales.cpu().numpy()
    want = (qo.reshape(8, -1, 8) * sw[:, None, None]).astype(np.float32).astype(np.float16).reshape(k.shape)
    exact = bool(np.array_equal(ch.repr_mask.cpu().numpy(), mask)
                 and np.array_equal(ch.packed.cpu().numpy(), O.pack_e8(qo[mask], 4))
                 and np.array_equal(out.cpu().numpy(), want))
    D = k.numel()
    V = D // 8
    v_in = int(mask.sum())
    P = 4 * v_in + 16 * (V - v_in) + (V + 7) // 8 + 2 * 8
    B = 4 * D + 2 * P
    # the device round trip gives the same mask, packed words and output
    cb = codec.compact_encode(kd, 4)
    dout = codec.compact_merge(cb)
    n_in = int(cb.totals[0])
    exact = exact and bool(np.array_equal(cb.mask.cpu().numpy().astype(bool), mask)
                           and np.array_equal(cb.packed[:n_in].cpu().numpy(), O.pack_e8(qo[mask], 4))
                           and np.array_equal(dout.cpu().numpy(), want))
    flush = CacheFlush(dev)
    dv = lambda: codec.compact_merge(codec.compact_encode(kd, 4), out=dout)
    rt = lambda: fused_decompress_chunk(compress_fixed_rate(kd, 4))
    ch_lb = dataclasses.replace(ch, tile_offsets=None)   # the merge then scans the mask itself
    exact = exact and bool(np.array_equal(fused_decompress_chunk(ch_lb).cpu().numpy(), want))
    mg = lambda: fused_decompress_chunk(ch_lb)
    mt = lambda: fused_decompress_chunk(ch)
    us_dv_f, us_dv_w = timed_median(dv, iters, flush), timed_median(dv, iters)
    us_rt_f, us_rt_w = timed_median(rt, iters, flush), timed_median(rt, iters)
    us_mg_f, us_mg_w = timed_median(mg, iters, flush), timed_median(mg, iters)
    us_mt_f = timed_median(mt, iters, flush)
    del flush
    return {"workload": "C1: K [1,8,2048,128] fp16 (randn seed 0, CPU), 4 b/d, compact 4-byte form + fp16 "
                        "fallback, no entropy coding", "input_sha256": sha, "bit_exact": exact,
            "in_range_frac": round(v_in / V, 4), "P_bytes": P, "B_bytes": B,
            "round_trip_flushed": _roof(B, us_dv_f, "compact_encode (sigma^2 partials; then scales, quantize, pack, "
                                                   "compact in one pass) + compact_merge, no host sync; 512 MiB "
                                                   "flush before each run"),
            "round_trip_warm": _roof(B, us_dv_w, "same, warm (MALL-resident working set)"),
            "api_round_trip_flushed": _roof(B, us_rt_f, "compress_fixed_rate + fused_decompress_chunk (one host "
                                                       "sync for the row counts), flushed"),
            "api_round_trip_warm": _roof(B, us_rt_w, "same, warm"),
            "merge_flushed": _roof(P + 2 * D, us_mg_f, "lq_fused_merge alone (reads P, writes 2 D; look-back "
                                                       "over the mask), flushed"),
            "merge_warm": _roof(P + 2 * D, us_mg_w, "lq_fused_merge alone, warm (MALL-resident)"),
            "merge_tile_offsets_flushed": _roof(P + 2 * D, us_mt_f, "lq_compact_merge with the encoder's tile "
                                                                   "offsets (a chunk from compress_fixed_rate), "
                                                                   "flushed")}


def _student_t(shape, g):
    """Student-t with nu = 3 from one CPU generator: z / sqrt(chi2_3 / 3),
    chi2_3 the sum of three squared standard normals."""
    z = torch.randn(shape, generator=g)
    c = torch.randn((3,) + tuple(shape), generator=g).square_().sum(0)
    return z / (c / 3.0).sqrt()


def make_c4():
    """C4 input, 28 layers of [1,4,16384,128] on the
    CPU: K Student-t(3) (generator seed 1000*layer) with 8 outlier channels per
    head (randperm(128)[:8] from the same generator, after the values) x20; V
    N(0,1) (seed 1000*layer + 1); fp16.  Bits per layer from
    allocation.eval_alloc.cyclic_schedule(28, seed=0): [3,4,5][l % 3].
    Returns (K list, V list, schedule, SHA-256 over K0 V0 K1 V1 ...)."""
    from latticequant_amd.allocation.eval_alloc import cyclic_schedule
    T = 16384
    sched = cyclic_schedule(28, seed=0)
    ks, vs = [], []
    h = hashlib.sha256()
    for layer in range(28):
        g = torch.Generator().manual_seed(1000 * layer)
        k = _student_t((4, T, HD), g)
        for hh in range(4):
            k[hh][:, torch.randperm(HD, generator=g)[:8]] *= 20.0
        v = torch.randn(4, T, HD, generator=torch.Generator().manual_seed(1000 * layer + 1))
        k16, v16 = k.half()[None], v.half()[None]
        h.update(memoryview(k16.numpy()).cast("B"))
        h.update(memoryview(v16.numpy()).cast("B"))
        ks.append(k16)
        vs.append(v16)
    return ks, vs, sched, h.hexdigest()


_SIDE_STREAMS = []


def side_streams(dev, n):
    """The first n side streams of the process (default priority), created
    once and shared by every leg.  HIP places a process's streams on its
    hardware queues (4 per process on these boxes) in creation order, so a leg
    that creates fresh streams after another leg's may find two of them on
    one queue, serialised; reusing the same streams keeps C4's three side
    streams on distinct queues whatever ran before."""
    while len(_SIDE_STREAMS) < n:
        _SIDE_STREAMS.append(torch.cuda.Stream(device=dev))
    return _SIDE_STREAMS[:n]


def bench_c4(dev, steps=5, n_streams=3):
    """C4: the 28-layer Qwen2.5-7B-shaped cache at its 3/4/5-bit schedule, one
    chunk per (layer, K/V), per-chunk tables, every chunk coded.  Chunks are
    grouped by rate (K on the int16 staging path, V on int8); the groups are
    independent and are dealt to n_streams streams (V groups first: their
    launches fill the chip while a K group's latency-bound table build runs
    beside them).  K coordinates whose stream alphabet exceeds L = 1024
    symbols (the reference's table normalisation never terminates there) are
    escaped: coarse symbols through the same tables and streams plus raw low
    bits (a format of this build).  The escape plan stays on the device; its
    C x 8 shifts reach the host when a K group's decode asks for them, so
    every group's encode is queued before the first K decode waits for its
    plan.  One step = encode every group + decode every group.  B = 4 D + 2 C
    over all chunks."""
    from latticequant_amd import codec
    from oracle import oracle as O
    ks_h, vs_h, sched, sha = make_c4()
    ks = [k.to(dev) for k in ks_h]
    vs = [v.to(dev) for v in vs_h]
    groups = []   # (x stacked (C,1,4,T,128), bits, wide)
    for r in (3, 4, 5):
        kl = [l for l in range(28) if sched[l]["K"] == r]
        vl = [l for l in range(28) if sched[l]["V"] == r]
        if kl:
            groups.append((torch.stack([ks[l] for l in kl]), r, True, [("K", l) for l in kl]))
        groups.append((torch.stack([vs[l] for l in vl]), r, False, [("V", l) for l in vl]))
    del ks, vs
    outs = [torch.empty_like(g[0]) for g in groups]
    arenas = [torch.empty(codec.words_bound(g[0].shape[0], g[0][0].numel() // 8), dtype=torch.int32, device=dev)
              for g in groups]
    encs = [None] * len(groups)
    side = side_streams(dev, n_streams) if n_streams > 1 else []
    order = sorted(range(len(groups)), key=lambda i: groups[i][2])   # int8 groups first

    def enc(i):
        x, r, wide, _ = groups[i]
        encs[i], _ = codec.encode_batch(x, r, exact_size=False, words_out=arenas[i], wide=wide)

    def dec(i):
        codec.decode_batch(encs[i], out=outs[i])

    def step():
        if not side:
            for i in order:
                enc(i)
                dec(i)
            return
        main = torch.cuda.current_stream(dev)
        for st in side:
            st.wait_stream(main)
        # group i always runs on the same stream; an int8 group is decoded
        # right after its encode, the wide groups only once every encode is
        # queued (their decode waits on the host for the escape plan)
        for j, i in enumerate(order):
            with torch.cuda.stream(side[j % len(side)]):
                enc(i)
                if not groups[i][2]:
                    dec(i)
        for j, i in enumerate(order):
            if groups[i][2]:
                with torch.cuda.stream(side[j % len(side)]):
                    dec(i)
        for st in side:
            main.wait_stream(st)

    step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True); e1 = torch.cuda.Event(enable_timing=True)
    gpu_busy()
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    st = int(np.bitwise_or.reduce(torch.cat([e.status for e in encs]).cpu().numpy()))
    D = sum(g[0].numel() for g in groups)
    Cb = sum(int(e.reference_bytes().sum() + e.side_bytes().sum()) for e in encs)
    B = 4 * D + 2 * Cb
    # parity: the first V chunk at 3 bits against the oracle's bitstream and decode;
    # every coded K chunk decodes to its lattice points times the fp16 scale (lossless)
    gi = next(i for i, g in enumerate(groups) if not g[2])
    e = encs[gi]
    x0 = groups[gi][0][0].cpu().numpy()
    ch = O.compress_chunk(x0, groups[gi][1], scales_f32=e.scale32.view(-1, 4)[0].cpu().numpy())
    nw = int(e.chunk_words[0])
    exact = bool(np.array_equal(e.words[:nw].cpu().numpy().view(np.uint32), ch.bitstream)
                 and np.array_equal(outs[gi][0].cpu().numpy(), O.decompress_chunk(ch)))
    lossless = True
    escaped = []
    for i, (x, r, wide, names) in enumerate(groups):
        if not wide:
            continue
        esc = encs[i].escape
        for c in range(x.shape[0]):
            q, _, _ = codec.quantize_points(x[c], r, scale32=encs[i].scale32.view(-1, 4)[c])
            want = (q.view(4, -1, 8) * encs[i].scale16.view(-1, 4)[c].float().view(4, 1, 1)).view(x[c].shape).half()
            lossless &= bool(torch.equal(outs[i][c], want))
            if esc is not None and esc.k_host[c].any():
                escaped.append((i, c, names[c][1]))
    # the first escaped K chunk against the oracle's restatement of the escape
    esc_exact = None
    if escaped:
        i, c, _ = escaped[0]
        e = encs[i]
        ch = O.compress_chunk(groups[i][0][c].cpu().numpy(), groups[i][1],
                              scales_f32=e.scale32.view(-1, 4)[c].cpu().numpy(), escape=True)
        base, nw = int(e.chunk_base[c]), int(e.chunk_words[c])
        fine = e.escape.fine.cpu().numpy().view(np.uint32)
        off = e.escape.off.cpu().numpy()
        esc_exact = bool(np.array_equal(e.words[base:base + nw].cpu().numpy().view(np.uint32), ch.bitstream)
                         and np.array_equal(e.escape.k_host[c], ch.esc_k)
                         and all(np.array_equal(fine[off[8 * c + j]:off[8 * c + j] + w.size], w)
                                 for j, w in ch.fine.items()))
    return {"workload": "C4: 28 layers x K,V x [1,4,16384,128] fp16, K Student-t(3) + 8 outlier channels x20, "
                        "V N(0,1), bits [3,4,5][l % 3], per-chunk tables",
            "input_sha256": sha, "chunks_coded": sum(g[0].shape[0] for g in groups), "chunks_total": 56,
            "k_layers_escaped": sorted(l for _, _, l in escaped), "status_flags": st,
            "bit_exact_v_chunk": exact, "k_chunks_lossless": lossless,
            "escaped_k_chunk_equals_oracle_escape": esc_exact,
            "step_us": round(us, 1), "streams": max(n_streams, 1), "D": D, "compressed_bytes": Cb,
            "effective_bits_per_dim": round(8 * Cb / D, 4),
            "roofline": _roof(B, us, "encode + decode of every coded chunk, B = 4 D + 2 C over them")}


def bench_c5(dev, layers):
    """C5: batch 8 x 131072 tokens of the
    Llama-3.1-8B shape, `layers` layers x K,V, one [8,8,131072,128] fp16 chunk
    per (layer, K/V), all resident in HBM; per-vector HeadRHT (seed
    layer*10000 + head*10 + kv) and subtractive dither, 4 bits/dim.  Inputs:
    torch.randn(fp32, device generator seeded 1000*layer + kv).half() (the CPU
    generator would take minutes at 137 GB), hashed on the host chunk by
    chunk.  Sustained write: encode_rotated of every chunk back to back
    (exact-size arenas: one size read-back per chunk); sustained read:
    decode_rotated of every chunk into two alternating fp16 buffers.  Bytes
    2 D + C per direction."""
    from concurrent.futures import ThreadPoolExecutor
    from latticequant_amd.llm import rotated as R
    shape = (1, 8, 8, 131072, HD)
    free, _ = torch.cuda.mem_get_info(dev)
    per_layer = 2 * (2 << 30) * 1.4     # two 2 GiB inputs + their chunks, blocks and staging
    fit = int((free - (24 << 30)) // per_layer)
    if fit < layers:
        print(f"[bench] C5: {free / 2**30:.0f} GiB free holds {fit} layers, not {layers}", file=sys.stderr, flush=True)
        layers = max(1, fit)
    n = 2 * layers
    xs, names = [], []
    shas = [None] * n
    pool = ThreadPoolExecutor(max_workers=max(1, min(8, len(os.sched_getaffinity(0)))))
    futs = []
    for layer in range(layers):
        for kv in range(2):
            g = torch.Generator(device=dev).manual_seed(1000 * layer + kv)
            x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32).half()
            xs.append(x)
            names.append((layer, kv))
            if len(futs) >= 8:
                futs.pop(0).result()
            futs.append(pool.submit(lambda i, h: shas.__setitem__(i, _sha(h)), len(xs) - 1, x.cpu()))
    for f in futs:
        f.result()
    pool.shutdown()
    sha = hashlib.sha256("".join(shas).encode()).hexdigest()
    outs = [torch.empty(shape, dtype=torch.float16, device=dev) for _ in range(2)]
    for i, x in enumerate(xs):   # each (layer, K/V)'s HeadRHT signs, drawn once as the reference's HeadRHT does
        R.prepare_signs(x.shape, [names[i][0]], [names[i][1]], dev)
    enc0, _ = R.encode_rotated(xs[0], BITS, [0], [0], exact_size=True, wide=False)   # warm-up
    R.decode_rotated(enc0, out=outs[0])
    del enc0
    torch.cuda.synchronize()
    encs = [None] * n
    e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    gpu_busy()
    e[0].record()
    for i, x in enumerate(xs):
        encs[i], _ = R.encode_rotated(x, BITS, [names[i][0]], [names[i][1]], exact_size=True, wide=False)
    e[1].record()
    for i in range(n):
        R.decode_rotated(encs[i], out=outs[i & 1])
    e[2].record()
    torch.cuda.synchronize()
    w_us, r_us = e[0].elapsed_time(e[1]) * 1e3, e[1].elapsed_time(e[2]) * 1e3
    st = int(np.bitwise_or.reduce(torch.cat([en.status for en in encs]).cpu().numpy()))
    D = sum(x.numel() for x in xs)
    Cb = sum(int(en.reference_bytes().sum() + en.side_bytes().sum()) for en in encs)
    # size-independent check on the last chunk: subtractive-dither error per head
    # = G(E8) a^2 (uniform on the scaled Voronoi cell), mean ~ 0
    y = outs[(n - 1) & 1]
    err = y.float() - xs[-1].float()
    sc = encs[-1].scale16.float().view(8, 8)
    mse = (err * err).mean(dim=(3, 4))[0] / (sc * sc)
    props = {"mse_over_G_scale2_min": round(float((mse / R.G_E8).min()), 4),
             "mse_over_G_scale2_max": round(float((mse / R.G_E8).max()), 4),
             "mean_err": float(err.mean())}
    del err, y
    return {"workload": f"C5: {layers} layers x K,V x [8,8,131072,128] fp16 resident ({D * 2 / 1e9:.1f} GB), "
                        "HeadRHT + subtractive dither, 4 b/d, one chunk per (layer, K/V)",
            "layers": layers, "chunks": n, "input_sha256_of_chunk_sha256s": sha, "status_flags": st,
            "D": D, "compressed_bytes": Cb, "effective_bits_per_dim": round(8 * Cb / D, 4),
            "dither_error_check": props,
            "write": _roof(2 * D + Cb, w_us, "encode_rotated of every chunk back to back, B = 2 D + C"),
            "read": _roof(2 * D + Cb, r_us, "decode_rotated of every chunk back to back, B = C + 2 D")}


def bench_decode_step(dev, iters=30, prefix=32768, tail=128):
    """C3: one decode step of Llama-3.1-8B GQA attention
    (32 q heads, 8 kv heads, head_dim 128) over a 32768-token E8+rANS prefix at
    4 bits/dim plus a 128-token fp16 tail.

    The prefix is compressed by the chunk codec (its rANS chunks are the at-rest
    form) and held resident as the same lattice points in the fixed-width form
    lq_resident_attention reads (b = 5 code words + exceptions).  Per iteration a
    512 MiB read evicts everything from L2 / MALL first (CacheFlush) and a
    queued GPU spin keeps host submission out of the events, so the step reads
    from HBM; also reported: after a 512 MiB write (dirty MALL lines) and warm.
    Also reported: the same step decoding the rANS chunks directly
    (lq_decode_attention).  Returns dict with the median step times and the
    roofline figures (algorithmic bytes C_K + C_V + tail + q + out)."""
    from latticequant_amd import codec
    from latticequant_amd.llm.decode_attention import attn_workspace as rans_workspace, decode_attention
    from latticequant_amd.llm.resident import attn_workspace, from_chunk, resident_decode_attention
    g = torch.Generator().manual_seed(3)
    k = torch.randn(1, 1, HEADS, prefix, HD, generator=g).half()
    v = torch.randn(1, 1, HEADS, prefix, HD, generator=g).half()
    q = torch.randn(1, 32, 1, HD, generator=g).half()
    tk = torch.randn(1, HEADS, tail, HD, generator=g).half()
    tv = torch.randn(1, HEADS, tail, HD, generator=g).half()
    sha = hashlib.sha256()
    for t in (k, v, q, tk, tv):
        sha.update(memoryview(t.numpy()).cast("B"))
    k, v, q, tk, tv = (t.to(dev) for t in (k, v, q, tk, tv))
    ek, _ = codec.encode_batch(k, BITS)
    ev, _ = codec.encode_batch(v, BITS)
    rk, rv = from_chunk(k[0], ek), from_chunk(v[0], ev)
    work = attn_workspace(HEADS, 4, prefix, tail, device=dev)
    out = resident_decode_attention(rk, rv, q, tk, tv, work=work)
    rwork = rans_workspace(ek, 4)
    out2 = decode_attention(ek, ev, q, tk, tv, work=rwork)
    flush = CacheFlush(dev)
    timed = lambda fn, n: timed_median(fn, n, flush)

    step = lambda: resident_decode_attention(rk, rv, q, tk, tv, work=work, out=out)
    us = timed(step, iters)
    us_dirty = timed_median(step, iters, CacheFlush(dev, write=True))
    us_warm = timed_median(step, iters)
    us_rans = timed(lambda: decode_attention(ek, ev, q, tk, tv, work=rwork, out=out2), max(5, iters // 3))
    cb = int(ek.reference_bytes().sum() + ek.side_bytes().sum() + ev.reference_bytes().sum() + ev.side_bytes().sum())
    small = tk.numel() * 2 + tv.numel() * 2 + q.numel() * 2 + out.numel() * 2
    nbytes = cb + small
    rbytes = rk.nbytes() + rv.nbytes() + small
    return {"decode_step_us": round(us, 2), "decode_step_bytes": nbytes,
            "decode_step_GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "decode_step_roofline_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "decode_step_resident_bytes_read": rbytes,
            "decode_step_resident_GBps": round(rbytes / (us * 1e-6) / 1e9, 1),
            "decode_tokens_per_s_32_layers": round(1e6 / (32 * us), 2),
            "decode_step_rans_direct_us": round(us_rans, 2),
            "decode_step_us_write_flush": round(us_dirty, 2),
            "decode_step_us_warm": round(us_warm, 2),
            "input_sha256": sha.hexdigest(),
            "decode_step_workload": f"C3: q [1,32,1,128], prefix K,V [1,8,{prefix},128] E8+rANS {BITS} b/d "
                                    f"(attention reads its resident b=5 form), tail [1,8,{tail},128] fp16, "
                                    f"L2/MALL flushed before each step"}


def e2e_decode_throughput(dev, prefills=(128, 8192), decode_tokens=64, warmup=2, repeats=3):
    """F1: model decode throughput through the HF cache interface, measured the
    way the reference measures it (llm/e2e_eval.py:285-362: prefill, then
    decode_tokens one-token forwards, tok/s over the decode phase), on a
    random-initialised model of the Llama-3.1-8B architecture (no weights are
    downloadable here), fp16.  Caches compared per prefill length:
      fp16      HF DynamicCache, SDPA over fp16 K / V (the reference's attention input)
      rans      CompressedKVCache (the reference's semantics: every update E8+rANS
                coded, decompressed fp16 K / V kept resident for SDPA)
      resident  ResidentKVCache: rANS chunks at rest + resident b=5 prefix +
                128-token fp16 tail; decode steps run lq_resident_attention"""
    from transformers import LlamaConfig, LlamaForCausalLM
    from transformers.cache_utils import DynamicCache
    from latticequant_amd.llm.compressed_kv_cache import CompressedKVCache
    from latticequant_amd.llm.resident_cache import ResidentKVCache, register
    name = register()
    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, rope_theta=500000.0,
                      max_position_embeddings=131072, attn_implementation=name)
    with torch.device("meta"):
        model = LlamaForCausalLM(cfg)
    model = model.to_empty(device=dev).to(torch.float16).eval()
    g = torch.Generator(device=dev).manual_seed(0)
    with torch.no_grad():
        for p_ in model.parameters():
            p_.normal_(0.0, 0.02, generator=g)
    for m in model.modules():   # RMSNorm weights to 1
        if hasattr(m, "variance_epsilon"):
            m.weight.data.fill_(1.0)
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    model.model.rotary_emb = LlamaRotaryEmbedding(cfg, device=dev)   # buffers were left empty on meta
    caches = {"fp16": lambda: DynamicCache(), "rans": lambda: CompressedKVCache(bits_per_dim=BITS),
              "resident": lambda: ResidentKVCache(bits_per_dim=BITS, tail_tokens=128)}
    res = {}
    for pre in prefills:
        ids = torch.randint(0, cfg.vocab_size, (1, pre), generator=g, device=dev)
        for label, mk in caches.items():
            ts = []
            for trial in range(warmup + repeats):
                cache = mk()
                with torch.no_grad():
                    out = model(ids, past_key_values=cache, use_cache=True)
                nxt = out.logits[:, -1:].argmax(-1)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                with torch.no_grad():
                    for _ in range(decode_tokens):
                        out = model(nxt, past_key_values=cache, use_cache=True)
                        nxt = out.logits[:, -1:].argmax(-1)
                torch.cuda.synchronize()
                if trial >= warmup:
                    ts.append(time.perf_counter() - t0)
                del cache, out
            t = float(np.mean(ts))
            res[f"{label}_prefill{pre}"] = {"tok_per_s": round(decode_tokens / t, 2),
                                             "ms_per_tok": round(t / decode_tokens * 1e3, 3)}
            print(f"e2e prefill {pre} {label}: {decode_tokens / t:.1f} tok/s", file=sys.stderr, flush=True)
    return res


def time_quantize(x, enc, reps=3):
    """Average duration (ms) of the k_chunk_quantize launch over the batch x
    (the launch encode_batch makes), with the scales enc holds, timed with
    events on the stream the kernel runs on; the histogram is cleared between
    launches, outside the events."""
    from latticequant_amd import _lib as L
    lib = L.lib()
    dev = x.device
    C = x.shape[0]
    nh, bph = HEADS, TOKENS * HD // 8
    nblk = (nh * bph + L.LQ_BLK - 1) // L.LQ_BLK
    s = L.stream_ptr(dev)
    fastdiv = torch.empty(C * nh, dtype=torch.int32, device=dev)
    L.check(lib.lq_scale_fastdiv(enc.scale32.data_ptr(), C * nh, L.dtype_code(x.dtype), fastdiv.data_ptr(), s),
            "lq_scale_fastdiv")
    sym = torch.empty(C * nblk * L.LQ_SYM_STRIDE, dtype=torch.int8, device=dev)
    coset = torch.empty(C * nblk * L.LQ_BLK // 8, dtype=torch.uint8, device=dev)
    n1 = torch.empty(C * nblk, dtype=torch.int32, device=dev)
    hist = torch.empty(C * L.LQ_STREAMS * 256, dtype=torch.int32, device=dev)
    status = torch.zeros(C, dtype=torch.int32, device=dev)
    ms = []
    for _ in range(reps):
        hist.zero_()
        e0 = torch.cuda.Event(enable_timing=True); e1 = torch.cuda.Event(enable_timing=True)
        gpu_busy()
        e0.record()
        L.check(lib.lq_chunk_quantize(x.data_ptr(), L.dtype_code(x.dtype), C, nh, bph, enc.scale32.data_ptr(),
                                      fastdiv.data_ptr(), sym.data_ptr(), coset.data_ptr(), n1.data_ptr(),
                                      hist.data_ptr(), status.data_ptr(), None, 0, None, s), "lq_chunk_quantize")
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    return float(np.mean(ms))


def gpu_busy():
    """Queue a short spin on the stream so that the host has submitted the
    launches that follow before the start event is reached: the events then
    bracket GPU time only, not the host's submission latency."""
    torch.cuda._sleep(10_000_000)



def load_traffic():
    """HBM bytes per launch per kernel, from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter on a copy of known
    size); {} when absent."""
    p = os.path.join(ROOT, "profiles", "roofline_traffic.json")
    if not os.path.exists(p):
        return {}
    with open(p) as f:
        return json.load(f).get("bytes_per_launch", {})


def copy_calibration(dev, nbytes=1 << 30):
    """One plain device copy of nbytes (the PMC calibration kernel)."""
    a = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    a.fill_(1)
    b.copy_(a)
    torch.cuda.synchronize()


def _kernel_base(name: str) -> str:
    """Kernel name without return type, namespace, template arguments or parameters."""
    n = name.replace("(anonymous namespace)::", "")
    if n.startswith("void "):
        n = n[5:]
    return n.split("(")[0].split("<")[0].strip()


def summarize_pmc(fetch_csv, write_csv, out_path, calib_bytes=1 << 30):
    """Turn two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE, then
    WRITE_SIZE, KiB per dispatch) of a run that ends with --copy-calib into HBM
    bytes per launch: each counter is scaled by what it reads for the 1 GiB
    copy (the largest __amd_rocclr_copyBuffer dispatch).  Per kernel the
    dispatches with the largest grid (the full-batch launches) are averaged."""
    import pandas as pd
    vals, factors = {}, {}
    for ctr, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        df = pd.read_csv(path)
        df = df[df["Counter_Name"] == ctr]
        cp = df[df["Kernel_Name"].str.contains("copyBuffer")]
        factors[ctr] = float(cp["Counter_Value"].max()) * 1024.0 / calib_bytes
        df = df.assign(base=df["Kernel_Name"].map(_kernel_base))
        for name, d in df.groupby("base"):
            if not name.startswith("k_"):
                continue
            d = d[d["Grid_Size"] == d["Grid_Size"].max()]
            vals.setdefault(name, {})[ctr] = float(d["Counter_Value"].mean()) * 1024.0
            vals[name]["grid"] = int(d["Grid_Size"].max())
            vals[name]["dispatches"] = int(len(d))
    res = {"bytes_per_launch": {n: round(v["FETCH_SIZE"] / factors["FETCH_SIZE"] + v["WRITE_SIZE"] / factors["WRITE_SIZE"])
                                for n, v in vals.items() if "FETCH_SIZE" in v and "WRITE_SIZE" in v},
           "raw_bytes": vals, "copy_factor": factors, "calib_bytes": calib_bytes}
    with open(out_path, "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps(res))


def summarize_counters(counter_csv, simds=1024, xcds=8):
    """Per-kernel means of every counter in a rocprofv3 --pmc
    counter_collection.csv (the largest-grid dispatches of each kernel), as a
    markdown table, plus two issue figures where the counters are present.
    GRBM_GUI_ACTIVE comes summed over the XCDs (each has its own GRBM), so a
    launch's busy cycles at its actual clock are GRBM_GUI_ACTIVE / xcds:
      issue_frac = 4 SQ_INSTS_VALU / (simds x GRBM_GUI_ACTIVE / xcds): the share
                   of those cycles the launch's VALU instructions occupy at one
                   wave64 instruction per 4 cycles per SIMD (1.0 = issue bound);
      valu_busy  = the same with SQ_ACTIVE_INST_VALU (rocprof's VALUBusy)."""
    import pandas as pd
    df = pd.read_csv(counter_csv)
    df = df.assign(base=df["Kernel_Name"].map(_kernel_base))
    rows = {}
    for (name, ctr), d in df.groupby(["base", "Counter_Name"]):
        if not name.startswith("k_"):
            continue
        d = d[d["Grid_Size"] == d["Grid_Size"].max()]
        r = rows.setdefault(name, {"grid": int(d["Grid_Size"].max()), "dispatches": 0})
        per = d.groupby("Dispatch_Id")["Counter_Value"].sum() if "Dispatch_Id" in d else d["Counter_Value"]
        r[ctr] = float(per.mean())
        r["dispatches"] = max(r["dispatches"], int(len(per)))
    ctrs = sorted({c for r in rows.values() for c in r if c not in ("grid", "dispatches")})
    extra = []
    if {"SQ_INSTS_VALU", "GRBM_GUI_ACTIVE"} <= set(ctrs):
        extra.append("issue_frac")
    if {"SQ_ACTIVE_INST_VALU", "GRBM_GUI_ACTIVE"} <= set(ctrs):
        extra.append("valu_busy")
    print("| kernel | grid | dispatches | " + " | ".join(ctrs + extra) + " |")
    print("|---|---:|---:|" + "---:|" * (len(ctrs) + len(extra)))
    for name, r in sorted(rows.items()):
        vals = [f"{r.get(c, float('nan')):.4g}" for c in ctrs]
        g = r.get("GRBM_GUI_ACTIVE")
        if "issue_frac" in extra:
            vals.append(f"{4 * r.get('SQ_INSTS_VALU', 0) / (simds * g / xcds):.3f}" if g else "")
        if "valu_busy" in extra:
            vals.append(f"{4 * r.get('SQ_ACTIVE_INST_VALU', 0) / (simds * g / xcds):.3f}" if g else "")
        print(f"| {name} | {r['grid']} | {r['dispatches']} | " + " | ".join(vals) + " |")


def summarize_trace(trace_csv, top=16):
    """Per (kernel, grid size) launch counts and durations from a rocprofv3
    --kernel-trace kernel_trace.csv, as a markdown table (longest total first)."""
    import pandas as pd
    df = pd.read_csv(trace_csv)
    df["us"] = (df["End_Timestamp"] - df["Start_Timestamp"]) / 1e3
    df["kernel"] = df["Kernel_Name"].str.replace("(anonymous namespace)::", "", regex=False).str.slice(0, 60)
    df["Grid_Size"] = df["Grid_Size_X"] * df["Grid_Size_Y"] * df["Grid_Size_Z"]
    g = df.groupby(["kernel", "Grid_Size"])["us"].agg(["count", "sum", "mean", "min", "max"]).reset_index()
    g = g.sort_values("sum", ascending=False).head(top)
    print("| kernel | grid | launches | total us | avg us | min us | max us |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for _, r in g.iterrows():
        print(f"| {r['kernel']} | {r['Grid_Size']} | {r['count']} | {r['sum']:.1f} | {r['mean']:.1f} | "
              f"{r['min']:.1f} | {r['max']:.1f} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 20 timed steps after 5 warm-up steps: shorter runs read the first steps
    # of a cold GPU (clocks still ramping: 2.02 against 1.90 ms per C2 step)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--group", type=int, default=64, help="chunks per kernel launch in the timed step")
    ap.add_argument("--streams", type=int, default=1,
                    help="streams the chunk groups of a step are dealt to (measured: one 64-chunk group on one "
                         "stream is fastest; concurrent groups do not overlap usefully)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-chunks", type=int, default=6,
                    help="C2 chunks the single-thread oracle codes (each also checked bit for bit)")
    ap.add_argument("--skip", default="", help="comma list of legs to leave out of the default run: c1,c3,c4,c5")
    ap.add_argument("--only", choices=["c1", "c3", "c4", "c5"],
                    help="run one leg alone and print its JSON (the profiling entry points)")
    ap.add_argument("--c5-layers", type=int, default=32, help="layers of the C5 cache (x K,V chunks of 2 GiB)")
    ap.add_argument("--c4-streams", type=int, default=3, help="streams the C4 rate groups are dealt to (1: one stream)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run one 1 GiB device copy (the HBM-counter calibration kernel under rocprofv3 --pmc)")
    ap.add_argument("--summarize-pmc", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "OUT_JSON"),
                    help="only summarise two rocprofv3 --pmc runs into per-launch HBM traffic and exit")
    ap.add_argument("--e2e", action="store_true",
                    help="only measure model decode tok/s through the HF cache interface (random-init Llama-3.1-8B "
                         "architecture; fp16, rANS and resident caches) and print one JSON line")
    ap.add_argument("--summarize-trace", metavar="KERNEL_TRACE_CSV",
                    help="only print per-(kernel, grid) launch durations of a rocprofv3 --kernel-trace run and exit")
    ap.add_argument("--summarize-counters", metavar="COUNTER_CSV",
                    help="only print per-kernel means of the counters of a rocprofv3 --pmc run (and the VALU issue "
                         "share when SQ_INSTS_VALU / SQ_ACTIVE_INST_VALU and GRBM_GUI_ACTIVE are among them) and exit")
    args = ap.parse_args()
    if args.summarize_counters:
        summarize_counters(args.summarize_counters)
        return
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for {args.gpus}); "
              "the per-chunk work is independent and would shard by layer / K-V with no communication.",
              file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    from latticequant_amd import _lib as L
    L.lib()
    if args.e2e:
        r = e2e_decode_throughput(dev)
        print(json.dumps({"metric": "decode tok/s (1 GPU, batch 1, 64 decode tokens after the prefill)",
                          "unit": "tok/s", "higher_is_better": True, "n_gpus": 1, "data": "synthetic",
                          "dtype": "fp16", "config": {"model": "Llama-3.1-8B architecture, random weights",
                                                     "bits_per_dim": BITS}, "results": r}))
        return
    legs = {"c1": lambda: bench_c1(dev), "c3": lambda: bench_decode_step(dev), "c4": lambda: bench_c4(dev, n_streams=args.c4_streams),
            "c5": lambda: bench_c5(dev, args.c5_layers)}
    if args.only:
        res = legs[args.only]()
        if args.copy_calib:
            copy_calibration(dev)
        print(json.dumps(res))
        return
    skip = {v.strip() for v in args.skip.split(",") if v.strip()}

    from latticequant_amd import codec

    def progress(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    progress("C2 inputs (CPU generator)")
    x, x_sha = make_kv(dev)
    C = x.shape[0]
    G = args.group
    groups = [(i, min(i + G, C)) for i in range(0, C, G)]
    V = HEADS * TOKENS * HD // 8
    bound = codec.words_bound(G, V)
    arenas = [torch.empty(bound, dtype=torch.int32, device=dev) for _ in groups]
    out = torch.empty_like(x)
    NS = max(1, args.streams)
    streams = side_streams(dev, NS)
    luts = [torch.empty(G * L.LQ_STREAMS * L.LQ_L, dtype=torch.int32, device=dev) for _ in range(NS)]
    encs = [None] * len(groups)

    def write():
        for gi, (a, b) in enumerate(groups):
            encs[gi], _ = codec.encode_batch(x[a:b], BITS, exact_size=False, words_out=arenas[gi], wide=False)

    def read():
        for gi, (a, b) in enumerate(groups):
            codec.decode_batch(encs[gi], out=out[a:b], lut_work=luts[0])

    def step():
        """Write then read every chunk group; group gi runs on stream gi % NS
        (defaults: one group of all 64 chunks, one stream)."""
        cur = torch.cuda.current_stream(dev)
        for st in streams:
            st.wait_stream(cur)
        for gi, (a, b) in enumerate(groups):
            with torch.cuda.stream(streams[gi % NS]):
                encs[gi], _ = codec.encode_batch(x[a:b], BITS, exact_size=False, words_out=arenas[gi], wide=False)
                codec.decode_batch(encs[gi], out=out[a:b], lut_work=luts[gi % NS])
        for st in streams:
            cur.wait_stream(st)

    progress("C2 timed steps")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # separate write / read timing (outside the headline loop): each direction
    # `steps` times back to back behind a queued spin, so that the events
    # bracket GPU time as in the headline loop, not the host's submission of
    # the first launches after an idle GPU
    nrep = max(1, args.steps)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    gpu_busy()
    ev[0].record()
    for _ in range(nrep):
        write()
    ev[1].record()
    torch.cuda.synchronize()
    gpu_busy()
    ev[2].record()
    for _ in range(nrep):
        read()
    ev[3].record()
    torch.cuda.synchronize()
    t_write_ms, t_read_ms = ev[0].elapsed_time(ev[1]) / nrep, ev[2].elapsed_time(ev[3]) / nrep

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0 = torch.cuda.Event(enable_timing=True); e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = e0.elapsed_time(e1) / args.steps

    # accounting (outside the timed region)
    ref_bytes = sum(int(e.reference_bytes().sum()) for e in encs)
    side_bytes = sum(int(e.side_bytes().sum()) for e in encs)
    status = torch.cat([e.status for e in encs]).cpu().numpy()
    D = x.numel()
    Cb = ref_bytes + side_bytes
    B = 4 * D + 2 * Cb
    value = B / (ms_per_step * 1e-3) / 1e9

    # the chunks the CPU baseline codes, with the GPU's words and decoded output
    # of the same chunks for the bit-exact check
    ncpu = max(1, args.cpu_chunks)
    xs = [x[i, 0].cpu().numpy()[None] for i in range(ncpu)]
    scs = [encs[i // G].scale32.view(-1, HEADS)[i % G].cpu().numpy() for i in range(ncpu)]
    gw, go = [], []
    for i in range(ncpu):
        e = encs[i // G]
        base = int(e.chunk_base[i % G]); nw = int(e.chunk_words[i % G])
        gw.append(e.words[base:base + nw].cpu().numpy().view(np.uint32))
        go.append(out[i].cpu().numpy())

    # rooflines of the two largest kernels, each timed per launch with events on
    # its own stream: k_chunk_quantize (write) and k_chunk_decode (read, with
    # its k_chunk_lut table build); the longer one is the headline roofline
    # (measured on single launches over all 64 chunks, outside the step)
    progress("C2 per-kernel rooflines")
    renc = codec.encode_batch(x, BITS, exact_size=False, wide=False)[0]
    rluts = torch.empty(C * L.LQ_STREAMS * L.LQ_L, dtype=torch.int32, device=dev)
    dec_ms = []
    for _ in range(3):
        s0 = torch.cuda.Event(enable_timing=True); s1 = torch.cuda.Event(enable_timing=True)
        gpu_busy()
        s0.record(); codec.decode_batch(renc, out=out, lut_work=rluts); s1.record()
        torch.cuda.synchronize()
        dec_ms.append(s0.elapsed_time(s1))
    q_ms = time_quantize(x, renc)
    # algorithmic bytes (each kernel's share of B = 4 D + 2 C): decode reads the
    # stored chunk C and writes 16 B of fp16 per vector; the quantizer reads
    # 16 B of fp16 per vector and writes the coset bitmap (one bit per vector),
    # its part of C.  Its int8 symbol staging (8 B per vector, written here and
    # read back by the encoder) is an intermediate: it shows in `traffic`, not
    # in the algorithmic bytes.
    dec_bytes = 2 * C * V * 8 + int(renc.reference_bytes().sum() + renc.side_bytes().sum())
    q_bytes = C * V * 16 + C * V // 8
    traffic = load_traffic()
    kern = {
        "k_chunk_decode": {"ms": float(np.mean(dec_ms)), "bytes": dec_bytes,
                           "desc": f"k_chunk_decode (+k_chunk_lut), {C}-chunk launch, algorithmic bytes = stored chunk + 16 B fp16 out per vector"},
        "k_chunk_quantize": {"ms": q_ms, "bytes": q_bytes,
                             "desc": f"k_chunk_quantize, {C}-chunk launch, algorithmic bytes = 16 B fp16 in + 1 coset bit per vector"},
    }
    del renc, rluts
    roof = {}
    for name, k in kern.items():
        ach = k["bytes"] / (k["ms"] * 1e-3) / 1e9
        tr = traffic.get(name)
        roof[name] = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": int(tr) if tr is not None else None,
                      "kernel": k["desc"], "avg_launch_us": round(k["ms"] * 1e3, 1),
                      "algorithmic_bytes": int(k["bytes"])}
    dominant = max(kern, key=lambda n: kern[n]["ms"])
    if args.copy_calib:
        copy_calibration(dev)

    extra = {}
    if "c3" not in skip:
        progress("C3 decode step")
        extra["c3"] = bench_decode_step(dev)
    del encs, arenas, luts
    if "c1" not in skip:
        progress("C1 round trip")
        extra["c1"] = bench_c1(dev)
    if "c4" not in skip:
        progress("C4 28-layer schedule")
        extra["c4"] = bench_c4(dev, n_streams=args.c4_streams)
    if "c5" not in skip:
        del x, out
        torch.cuda.empty_cache()
        progress(f"C5 {args.c5_layers} layers")
        extra["c5"] = bench_c5(dev, args.c5_layers)
        torch.cuda.empty_cache()

    cpu, exact_idx, info = None, [], cpu_info()
    if not args.no_cpu_baseline:
        progress("CPU baselines")
        tiers, exact_idx, info = cpu_baseline(xs, BITS, scs, gw, go)
        cpu = dict(tiers["port"])
        cpu.update({"cpu_model": info["cpu_model"], "affinity_cores": info["affinity_cores"],
                    "torch_threads": info["torch_threads"], "tiers": tiers})
    else:
        from oracle import oracle as O
        for i in range(ncpu):
            ch = O.compress_chunk(xs[i], BITS, scales_f32=scs[i])
            if np.array_equal(gw[i], ch.bitstream) and np.array_equal(go[i], O.decompress_chunk(ch)):
                exact_idx.append(i)

    c3 = extra.get("c3") or {}
    res = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 quantize / u32 rANS (fp16 in, fp16 out)", "data": "synthetic",
        "config": {"workload": "C2: Llama-3.1-8B KV cache write+read, 32 layers x K,V x [1,8,8192,128] fp16, "
                               "N(0,1) + 4 outlier channels x10 per head, 4 bits/dim, one chunk per layer/K-V",
                   "chunks": C, "group": G, "streams": NS, "bits_per_dim": BITS},
        "input_sha256": x_sha,
        "write_ms": round(t_write_ms, 4), "read_ms": round(t_read_ms, 4),
        "write_GBps": round((2 * D + Cb) / (t_write_ms * 1e-3) / 1e9, 2),
        "read_GBps": round((2 * D + Cb) / (t_read_ms * 1e-3) / 1e9, 2),
        "compressed_bytes": Cb, "reference_accounting_bytes": ref_bytes, "side_info_bytes": side_bytes,
        "effective_bits_per_dim": round(8 * Cb / D, 4),
        "reference_bits_per_dim": round(8 * ref_bytes / D, 4),
        "status_flags": int(np.bitwise_or.reduce(status)),
        "bit_exact_chunks": f"{len(exact_idx)}/{ncpu}", "bit_exact": len(exact_idx) == ncpu,
        "roofline": roof[dominant],
        "roofline_other": {n: r for n, r in roof.items() if n != dominant},
        "cpu_baseline": cpu,
        "decode_step_us": c3.get("decode_step_us"),
        "decode_step": c3 or None,
        "c1": extra.get("c1"), "c4": extra.get("c4"), "c5": extra.get("c5"),
        "wall_s": round(wall, 3),
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
