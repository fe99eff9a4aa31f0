"""Write the golden input/output vectors that pin the CPU oracle.

Runs ONLY in the build container, where the reference checkout is mounted
read-only at /root/reference.  It imports the reference's own CPU functions,
feeds them seeded inputs and stores inputs + outputs as small ``.npz``
fixtures next to this script.  Nothing from the reference is stored except
these input/output arrays; the GPU box never needs the reference.

Functions exercised (reference file:line):
  core/e8_quantizer.py:20-83   encode_d8 / encode_e8 (fp32 near-ties, 1e-7 tiebreak)
  core/e8_quantizer.py:137-148 compute_scale
  core/entropy_coder.py:46-89  e8_to_symbols / symbols_to_e8
  core/compact_storage.py:87-222 pack_e8 / unpack_e8 (b = 3, 4, 5)
  core/gpu_ans.py:62-168       build_rans_table / rans_encode / rans_decode_cpu
  llm/compressed_kv_cache.py:46-63,176-287 pack_coset_bits, _compress_tensor
  core/pipeline.py:81-118      RHT sign vectors

Usage:  python tests/golden/make_golden.py      (writes tests/golden/*.npz)
"""
import json
import os
import sys

import numpy as np
import torch

REF = os.environ.get("LQ_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))


def _import_reference():
    sys.path.insert(0, os.path.join(REF, "core"))
    sys.path.insert(0, os.path.join(REF, "llm"))
    import e8_quantizer as e8q
    import entropy_coder as ec
    import compact_storage as cs
    import gpu_ans as ga
    import compressed_kv_cache as ckv
    import pipeline as pl
    return e8q, ec, cs, ga, ckv, pl


def e8_inputs(rng, e8q):
    """Seeded E8 inputs: Gaussian at b=3/4/5 scales, wide, dyadic ties, near ties."""
    parts = []
    for b in (3, 4, 5):
        a = e8q.compute_scale(1.0, b)
        parts.append((rng.standard_normal((4096, 8)) / a).astype(np.float32))
    parts.append((rng.standard_normal((2048, 8)) * 40.0).astype(np.float32))
    # dyadic grid points: exact .5 ties for round(), exact argmin ties, exact dist ties
    parts.append((rng.integers(-16, 17, size=(4096, 8)) / 4.0).astype(np.float32))
    parts.append((rng.integers(-8, 9, size=(2048, 8)) / 2.0).astype(np.float32))
    # flip-cost near ties: residuals that differ by ~1e-7
    base = rng.integers(-4, 5, size=(2048, 8)).astype(np.float32)
    r = np.float32(0.3) + (rng.integers(-3, 4, size=(2048, 8)) * 1e-7).astype(np.float32)
    sgn = np.where(rng.random((2048, 8)) < 0.5, -1, 1).astype(np.float32)
    parts.append((base + sgn * r).astype(np.float32))
    # D8 / D8+1/2 boundary: 0.25 offsets plus ulp-scale jitter
    base = rng.integers(-3, 4, size=(2048, 8)).astype(np.float32)
    jit = (rng.integers(-2, 3, size=(2048, 8)) * 2.0 ** -22).astype(np.float32)
    parts.append((base + np.float32(0.25) + jit).astype(np.float32))
    parts.append((base - np.float32(0.25) + jit).astype(np.float32))
    # tiny and signed zeros
    tiny = (rng.standard_normal((512, 8)) * 1e-6).astype(np.float32)
    tiny[::7, 3] = -0.0
    parts.append(tiny)
    return np.concatenate(parts, axis=0)


def gen_e8(rng, e8q, ec):
    x = e8_inputs(rng, e8q)
    xt = torch.from_numpy(x)
    d8 = e8q.encode_d8(xt.clone()).numpy()
    e8 = e8q.encode_e8(xt.clone()).numpy()
    coset, free, c8h = ec.e8_to_symbols(torch.from_numpy(e8))
    back = ec.symbols_to_e8(coset, free, c8h).numpy()
    scales = np.array([e8q.compute_scale(s2, b) for s2 in (1.0, 0.37, 12.5, 3e-5)
                       for b in (3, 4, 5)], dtype=np.float64)
    np.savez_compressed(os.path.join(HERE, "e8.npz"), x=x, d8=d8, e8=e8,
                        coset=coset.numpy(), free=free.numpy(), c8h=c8h.numpy(),
                        back=back, scales=scales)


def gen_compact(rng, e8q, cs):
    out = {}
    for b in (3, 4, 5):
        a = e8q.compute_scale(1.0, b)
        x = torch.from_numpy((rng.standard_normal((6000, 8))).astype(np.float32))
        q = e8q.encode_e8(x / a)
        ok = cs.check_representable(q, b)
        qr = q[ok]
        packed = cs.pack_e8(qr, b)
        out[f"q{b}"] = qr.numpy()
        out[f"packed{b}"] = packed.numpy()
        out[f"inrange{b}"] = ok.numpy()
        raw = torch.from_numpy(rng.integers(0, 256, size=(3000, b)).astype(np.uint8))
        out[f"raw{b}"] = raw.numpy()
        out[f"unpacked{b}"] = cs.unpack_e8(raw, b).numpy()
    np.savez_compressed(os.path.join(HERE, "compact.npz"), **out)


def _count_cases(rng):
    """Histograms for build_rans_table: tie-heavy synthetic + E8 column histograms."""
    cases = []
    # the reference's own test distributions (core/gpu_ans.py:390-405, 480-484)
    cases.append(np.array([1, 3, 10, 30, 50, 60, 50, 30, 10, 3, 1]))
    cases.append(np.array([500, 10, 3, 2, 1]))
    cases.append(np.array([13, 12, 13, 12, 13, 12, 13, 12]))
    cases.append(np.array([70, 30]))
    cases.append(np.array([1, 1, 1, 200, 1, 1, 1]))
    cases.append(np.array([max(1, int(50 * np.exp(-x ** 2 / 10))) for x in range(-15, 16)]))
    cases.append(np.array([5, 10, 20, 10, 5]))
    cases.append(np.array([5, 10, 20, 50, 20, 10, 5]))
    cases.append(np.array([200, 20, 5, 1]))
    cases.append(np.zeros(5))                       # empty histogram
    cases.append(np.array([0, 0, 7, 0, 0]))         # single symbol
    for _ in range(600):
        n = int(rng.integers(2, 120))
        kind = rng.integers(0, 4)
        if kind == 0:
            c = rng.integers(0, 4, size=n)
        elif kind == 1:
            c = rng.integers(0, 3, size=n) * int(rng.integers(1, 50))
        elif kind == 2:
            g = np.exp(-((np.arange(n) - n / 2) ** 2) / max(1.0, n * rng.random()))
            c = np.round(g * rng.integers(10, 100000)).astype(np.int64)
        else:
            c = rng.integers(0, 2000, size=n)
        cases.append(np.asarray(c))
    for n in (200, 256, 300, 600, 1000):
        cases.append(rng.integers(0, 5, size=n))
    return [np.asarray(c, dtype=np.int64) for c in cases]


def gen_rans(rng, ga, e8q, ec):
    cases = _count_cases(rng)
    # E8 column histograms as the cache builds them (llm/compressed_kv_cache.py:242-248)
    cols = []
    for b in (3, 4, 5):
        a = e8q.compute_scale(1.0, b)
        for nvec in (64, 700, 5000):
            x = torch.from_numpy(rng.standard_normal((nvec, 8)).astype(np.float32))
            q = e8q.encode_e8(x / a)
            coset, free, c8h = ec.e8_to_symbols(q)
            syms = np.concatenate([free.numpy(), c8h.numpy()[:, None]], 1)
            cn = coset.numpy()
            for c in (0, 1):
                sc = syms[cn == c]
                if len(sc) == 0:
                    continue
                for i in range(8):
                    col = sc[:, i]
                    u, uc = np.unique(col, return_counts=True)
                    lo = int(u.min()) - 2
                    alph = np.arange(lo, int(u.max()) + 3)
                    cnt = np.zeros(len(alph), dtype=np.int64)
                    cnt[u - lo] = uc
                    cases.append(cnt)
                    cols.append((lo, col.astype(np.int64)))
    tab_counts, tab_lo, tab_freqs, tab_lookup = [], [], [], []
    for i, cnt in enumerate(cases):
        lo = -(len(cnt) // 2)
        alph = list(range(lo, lo + len(cnt)))
        t = ga.build_rans_table(cnt.copy(), alph)
        tab_counts.append(cnt)
        tab_lo.append(lo)
        tab_freqs.append(np.asarray(t.freqs, dtype=np.int32))
        tab_lookup.append(np.asarray(t.lookup, dtype=np.int32))
    # encode streams: E8 columns with their own tables, plus synthetic streams
    enc_syms, enc_lo, enc_counts, enc_words, enc_state, enc_nbits = [], [], [], [], [], []
    for lo, col in cols:
        u, uc = np.unique(col, return_counts=True)
        alph = list(range(lo, int(u.max()) + 3))
        cnt = np.zeros(len(alph), dtype=np.int64)
        cnt[u - lo] = uc
        t = ga.build_rans_table(cnt.copy(), alph)
        words, st, nb = ga.rans_encode(col, t)
        dec = ga.rans_decode_cpu(words, nb, st, t, len(col))
        assert np.array_equal(dec, col)
        enc_syms.append(col); enc_lo.append(lo); enc_counts.append(cnt)
        enc_words.append(np.asarray(words, dtype=np.uint32)); enc_state.append(st); enc_nbits.append(nb)
    for k in range(40):
        n_sym = int(rng.integers(5, 40))
        lo = int(rng.integers(-20, 0))
        alph = list(range(lo, lo + n_sym))
        p = rng.random(n_sym) ** 3
        cnt = np.maximum((p / p.sum() * 1000).astype(np.int64), 0)
        length = int(rng.integers(0, 3000)) if k % 5 else int(rng.integers(0, 4))
        pp = (cnt + 1e-3) / (cnt + 1e-3).sum()
        col = rng.choice(np.array(alph), size=length, p=pp).astype(np.int64)
        t = ga.build_rans_table(cnt.copy(), alph)
        words, st, nb = ga.rans_encode(col, t)
        enc_syms.append(col); enc_lo.append(lo); enc_counts.append(cnt)
        enc_words.append(np.asarray(words, dtype=np.uint32)); enc_state.append(st); enc_nbits.append(nb)

    def ragged(arrs, dtype):
        offs = np.zeros(len(arrs) + 1, dtype=np.int64)
        offs[1:] = np.cumsum([len(a) for a in arrs])
        flat = np.concatenate([np.asarray(a, dtype=dtype) for a in arrs]) if arrs else np.zeros(0, dtype)
        return flat, offs

    out = {}
    out["tab_counts"], out["tab_counts_off"] = ragged(tab_counts, np.int64)
    out["tab_freqs"], _ = ragged(tab_freqs, np.int32)
    out["tab_lookup"] = np.stack(tab_lookup)
    out["tab_lo"] = np.array(tab_lo, dtype=np.int64)
    out["enc_syms"], out["enc_syms_off"] = ragged(enc_syms, np.int64)
    out["enc_counts"], out["enc_counts_off"] = ragged(enc_counts, np.int64)
    out["enc_words"], out["enc_words_off"] = ragged(enc_words, np.uint32)
    out["enc_lo"] = np.array(enc_lo, dtype=np.int64)
    out["enc_state"] = np.array(enc_state, dtype=np.int64)
    out["enc_nbits"] = np.array(enc_nbits, dtype=np.int64)
    np.savez_compressed(os.path.join(HERE, "rans.npz"), **out)


def gen_cache(rng, ckv, ga, ec):
    """One CompressedKVCache._compress_tensor per case on CPU tensors."""
    cases = [((1, 2, 64, 128), 4, 0), ((1, 2, 64, 128), 3, 1), ((1, 2, 64, 128), 5, 2),
             ((2, 2, 32, 64), 4, 3), ((1, 1, 16, 72), 4, 4), ((1, 2, 40, 128), 4, 5),
             ((1, 1, 8, 16), 4, 6)]
    out = {}
    for ci, (shape, bits, seed) in enumerate(cases):
        g = torch.Generator().manual_seed(1234 + seed)
        t = torch.randn(*shape, generator=g).to(torch.float16)
        if seed == 5:
            t[:, :, :, 3] *= 10.0          # outlier channel
        if seed == 6:
            t[:, :, :, :] = 0.0            # all-zero head -> sigma2 < 1e-12 -> scale 1
        cache = ckv.CompressedKVCache(bits_per_dim=bits)
        chunk, dec = cache._compress_tensor(t)
        # rebuild through the reference's own CPU decoder (the Triton decoder needs CUDA)
        n = chunk.n_vectors
        cos = np.array([(int(chunk.coset_packed[i // 8]) >> (i % 8)) & 1 for i in range(n)], dtype=np.int64)
        syms = np.zeros((n, 8), dtype=np.int64)
        si = 0
        for c in (0, 1):
            rows = np.where(cos == c)[0]
            if len(rows) == 0:
                continue
            for idx in range(8):
                s = chunk.streams[si]
                syms[rows, idx] = ga.rans_decode_cpu(s.bitstream, s.n_bits, s.initial_state, s.table, s.n_symbols)
                si += 1
        q = ec.symbols_to_e8(torch.from_numpy(cos), torch.from_numpy(syms[:, :7]), torch.from_numpy(syms[:, 7]))
        qh = q.reshape(chunk.n_heads, chunk.blocks_per_head, 8)
        rec = torch.zeros_like(qh)
        for h in range(chunk.n_heads):
            rec[h] = qh[h] * chunk.scales[h].float().item()
        rec = rec.reshape(shape).to(torch.float16)
        p = f"c{ci}_"
        out[p + "input"] = t.numpy()
        out[p + "bits"] = np.array(bits)
        out[p + "decompressed"] = dec.numpy()
        out[p + "rebuilt"] = rec.numpy()
        out[p + "scales"] = chunk.scales.numpy()
        out[p + "coset_packed"] = chunk.coset_packed.numpy()
        out[p + "coset_counts"] = np.array(chunk.coset_counts)
        out[p + "bitstream"] = chunk.gpu_bitstream.numpy().view(np.uint32)
        out[p + "word_offsets"] = np.array(chunk.stream_word_offsets, dtype=np.int64)
        out[p + "stream_meta"] = np.array(chunk.stream_meta, dtype=np.int64).reshape(-1, 3)
        out[p + "states"] = np.array([s.initial_state for s in chunk.streams], dtype=np.int64)
        out[p + "nbits"] = np.array([s.n_bits for s in chunk.streams], dtype=np.int64)
        out[p + "alpha_lo"] = np.array([s.table.alphabet[0] for s in chunk.streams], dtype=np.int64)
        fr, offs = [], [0]
        for s in chunk.streams:
            fr.append(np.asarray(s.table.freqs, dtype=np.int32))
            offs.append(offs[-1] + len(s.table.freqs))
        out[p + "freqs"] = np.concatenate(fr) if fr else np.zeros(0, np.int32)
        out[p + "freqs_off"] = np.array(offs, dtype=np.int64)
        out[p + "compressed_bytes"] = np.array(chunk.gpu_bitstream.nelement() * 4
                                               + chunk.coset_packed.nelement()
                                               + chunk.scales.nelement() * 2)
    out["n_cases"] = np.array(len(cases))
    # uncompressible passthrough (hd % 8 != 0)
    cache = ckv.CompressedKVCache(bits_per_dim=4)
    t = torch.randn(1, 2, 4, 12, generator=torch.Generator().manual_seed(9)).to(torch.float16)
    r, d = cache._compress_tensor(t)
    out["uncompressible_tag"] = np.array(r == "uncompressible")
    np.savez_compressed(os.path.join(HERE, "cache.npz"), **out)


def gen_rht(pl):
    seeds = [0, 1, 7, 10000 * 3 + 10 * 5 + 1, 10000 * 31 + 10 * 7 + 0, 123456]
    signs = np.stack([pl.RHT(128, seed=s).signs.numpy() for s in seeds])
    x = torch.randn(16, 128, generator=torch.Generator().manual_seed(5))
    y = pl.RHT(128, seed=7).forward(x.clone())
    np.savez_compressed(os.path.join(HERE, "rht.npz"), seeds=np.array(seeds), signs=signs,
                        x=x.numpy(), y=y.numpy())


def gen_allocation():
    """The reference's published Qwen2.5-7B 4-bit allocation (results/*.json,
    data only): the per-layer fields allocation_to_schedule reads."""
    src = os.path.join(REF, "results", "allocation_Qwen2.5-7B_4b.json")
    with open(src) as f:
        d = json.load(f)
    keep = {"model": d["model"], "n_layers": d["n_layers"], "budget_discrete": d["budget_discrete"],
            "layers": [{k: lr[k] for k in ("layer", "b_K", "b_V", "b_K_disc", "b_V_disc")} for lr in d["layers"]]}
    with open(os.path.join(HERE, "allocation_Qwen2.5-7B_4b.json"), "w") as f:
        json.dump(keep, f, indent=0)


def main():
    gen_allocation()
    e8q, ec, cs, ga, ckv, pl = _import_reference()
    rng = np.random.default_rng(20261201)
    gen_e8(rng, e8q, ec)
    gen_compact(rng, e8q, cs)
    gen_rans(rng, ga, e8q, ec)
    gen_cache(rng, ckv, ga, ec)
    gen_rht(pl)
    meta = {
        "torch": torch.__version__,
        "numpy": np.__version__,
        "cpu_capability": torch.backends.cpu.get_cpu_capability(),
        "torch_threads": torch.get_num_threads(),
        "reference": "yoon9728/LatticeQuant (read-only checkout)",
    }
    with open(os.path.join(HERE, "meta.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("golden fixtures written:", sorted(p for p in os.listdir(HERE) if p.endswith(".npz")))


if __name__ == "__main__":
    main()
