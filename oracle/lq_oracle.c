/*
 * lq_oracle.c -- CPU restatement of LatticeQuant's compressed-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU path is compared
 * against; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product (latticequant_amd) never calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the yoon9728/LatticeQuant checkout).  Built with
 * -ffp-contract=off so that every fp32 operation rounds exactly where the
 * reference's torch ops round.
 *
 * Pinning (what checks each function, besides the golden vectors written by
 * tests/golden/make_golden.py from the reference itself):
 *   lqo_encode_d8/e8    brute-force nearest point on tiny inputs, E8 validity
 *   lqo_argsort         numpy.argsort on an AVX512 host, exhaustive small n
 *   lqo_build_table     sum == L, freqs >= 1, golden tables
 *   lqo_rans_encode     decode(encode(s)) == s, golden bitstreams
 *   lqo_pack/unpack     known-answer points of the reference test, round trip
 *   lqo_dither          build-defined (the reference has no E8 dither):
 *                       SplitMix64 known-answer values, range [-1, 1), mean
 *                       and variance 1/3 per coordinate, and the subtractive-
 *                       dither error being uniform on the E8 Voronoi cell
 *                       (per-dimension MSE G(E8) = 0.07168, zero mean)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define LQO_L 1024
#define LQO_LOG2_L 10

/* ------------------------------------------------------------------ E8 --- */

/* tiebreaker of encode_d8: torch.arange(8, dtype=f32) * 1e-7, i.e. RN32(i * f32(1e-7))
 * (core/e8_quantizer.py:42-44) */
static float tiebreak(int i) { return (float)i * 1e-7f; }

/* encode_d8 for one 8-vector (core/e8_quantizer.py:20-58). */
static void d8_one(const float *x, float *r) {
    float res[8], best = 0.f;
    int idx = 0;
    float s = 0.f;
    for (int i = 0; i < 8; i++) {
        r[i] = rintf(x[i]);               /* torch.round: half to even */
        s += r[i];                        /* integer-valued: order irrelevant */
    }
    for (int i = 0; i < 8; i++) {
        res[i] = x[i] - r[i];
        float two = 2.0f * fabsf(res[i]);
        float fc = 1.0f - two;            /* flip_cost */
        float adj = fc + tiebreak(i);     /* flip_cost_adj */
        if (i == 0 || adj < best) { best = adj; idx = i; }   /* argmin: first index */
    }
    int64_t si = (int64_t)s;
    if (si & 1) {                          /* parity = sum % 2 != 0 */
        float sg = res[idx] > 0.f ? 1.f : (res[idx] < 0.f ? -1.f : 1.f); /* sign, 0 -> +1 */
        r[idx] += sg;
    }
}

void lqo_encode_d8(const float *x, float *out, int64_t n) {
    for (int64_t v = 0; v < n; v++) d8_one(x + 8 * v, out + 8 * v);
}

/* encode_e8 (core/e8_quantizer.py:61-83).  The two squared distances are summed
 * left to right, which is the order torch's CPU sum(dim=-1) uses for 8-wide rows
 * (checked against torch in tests/test_oracle.py). */
static void e8_one(const float *x, float *out) {
    float c1[8], c2[8], y[8];
    d8_one(x, c1);
    for (int i = 0; i < 8; i++) y[i] = x[i] - 0.5f;
    d8_one(y, c2);
    for (int i = 0; i < 8; i++) c2[i] = c2[i] + 0.5f;
    float d1 = 0.f, d2 = 0.f;
    for (int i = 0; i < 8; i++) {
        float a = x[i] - c1[i];
        float b = x[i] - c2[i];
        float a2 = a * a, b2 = b * b;
        d1 = (i == 0) ? a2 : d1 + a2;
        d2 = (i == 0) ? b2 : d2 + b2;
    }
    const float *c = (d1 <= d2) ? c1 : c2;
    for (int i = 0; i < 8; i++) out[i] = c[i];
}

void lqo_encode_e8(const float *x, float *out, int64_t n) {
    for (int64_t v = 0; v < n; v++) e8_one(x + 8 * v, out + 8 * v);
}

/* x / scale[head] then encode_e8, as _compress_tensor does
 * (llm/compressed_kv_cache.py:199-201).  x is fp32, n_heads*bph vectors. */
void lqo_quantize_heads(const float *x, const float *scale, int64_t n_heads, int64_t bph,
                        float *q) {
    float t[8];
    for (int64_t h = 0; h < n_heads; h++) {
        float s = scale[h];
        for (int64_t v = 0; v < bph; v++) {
            const float *xv = x + 8 * (h * bph + v);
            for (int i = 0; i < 8; i++) t[i] = xv[i] / s;
            e8_one(t, q + 8 * (h * bph + v));
        }
    }
}

/* ------------------------------------------------------------- dither --- */

/* SplitMix64 output function (Steele, Lea, Flood, "Fast splittable
 * pseudorandom number generators", OOPSLA 2014). */
uint64_t lqo_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Dither of vectors v0 .. v0 + n - 1 of a chunk with seed `seed`: coordinates
 * 4p .. 4p + 3 from the four 16-bit fields (least significant first) of
 * mix64(mix64(seed) + 2 v + p), p = 0, 1, each (k - 2^15) * 2^-15 in [-1, 1). */
void lqo_dither(int64_t seed, int64_t v0, int64_t n, float *d) {
    const uint64_t key = lqo_mix64((uint64_t)seed);
    for (int64_t v = 0; v < n; v++) {
        for (int p = 0; p < 2; p++) {
            const uint64_t h = lqo_mix64(key + (uint64_t)(v0 + v) * 2u + (uint64_t)p);
            for (int j = 0; j < 4; j++)
                d[8 * v + 4 * p + j] = (float)((int32_t)((h >> (16 * j)) & 0xFFFFu) - (1 << 15)) * 0x1p-15f;
        }
    }
}

/* lqo_quantize_heads with the subtractive dither added to x / scale. */
void lqo_quantize_heads_dither(const float *x, const float *scale, int64_t n_heads, int64_t bph, int64_t seed,
                               float *q) {
    float t[8], d[8];
    for (int64_t h = 0; h < n_heads; h++) {
        float s = scale[h];
        for (int64_t v = 0; v < bph; v++) {
            const float *xv = x + 8 * (h * bph + v);
            lqo_dither(seed, h * bph + v, 1, d);
            for (int i = 0; i < 8; i++) t[i] = xv[i] / s + d[i];
            e8_one(t, q + 8 * (h * bph + v));
        }
    }
}

/* e8_to_symbols (core/entropy_coder.py:46-68): coset, 7 free coords, floor(c7/2). */
void lqo_e8_to_symbols(const float *q, int64_t n, int32_t *coset, int32_t *sym8) {
    for (int64_t v = 0; v < n; v++) {
        const float *p = q + 8 * v;
        int half = fabsf(p[0] - rintf(p[0])) > 0.25f;
        coset[v] = half;
        for (int i = 0; i < 8; i++) {
            float t = half ? p[i] - 0.5f : p[i];
            int32_t ic = (int32_t)rintf(t);
            sym8[8 * v + i] = (i < 7) ? ic : (int32_t)floor((double)ic / 2.0);
        }
    }
}

static int32_t floormod2(int64_t a) { return (int32_t)(((a % 2) + 2) % 2); }

/* symbols_to_e8 (core/entropy_coder.py:71-89). */
void lqo_symbols_to_e8(const int32_t *coset, const int32_t *sym8, int64_t n, float *q) {
    for (int64_t v = 0; v < n; v++) {
        const int32_t *s = sym8 + 8 * v;
        int64_t sum7 = 0;
        for (int i = 0; i < 7; i++) sum7 += s[i];
        int64_t c7 = 2 * (int64_t)s[7] + floormod2(sum7);
        float off = coset[v] == 1 ? 0.5f : 0.f;
        for (int i = 0; i < 7; i++) q[8 * v + i] = (float)s[i] + off;
        q[8 * v + 7] = (float)c7 + off;
    }
}

/* pack_coset_bits (llm/compressed_kv_cache.py:46-54): bit i -> byte i/8, bit i%8. */
void lqo_pack_coset_bits(const int32_t *coset, int64_t n, uint8_t *out) {
    memset(out, 0, (size_t)((n + 7) / 8));
    for (int64_t i = 0; i < n; i++) out[i / 8] |= (uint8_t)((coset[i] & 1) << (i % 8));
}

/* --------------------------------------------------------- compact form --- */

/* pack_e8 (core/compact_storage.py:87-154), one vector of already validated,
 * in-range integer coords.  Returns 0, or -1 if out of range. */
int lqo_pack_e8(const float *q, int64_t n, int bits, uint8_t *out) {
    int64_t R = 1LL << (bits - 1);
    for (int64_t v = 0; v < n; v++) {
        const float *p = q + 8 * v;
        int half = fabsf((p[0] - 0.5f) - rintf(p[0] - 0.5f)) < 1e-5f;
        int64_t u[8];
        for (int i = 0; i < 8; i++) {
            float t = half ? p[i] - 0.5f : p[i];
            int64_t ic = (int64_t)rintf(t);
            if (ic < -R || ic > R - 1) return -1;
            u[i] = ic + R;
        }
        uint64_t w = (uint64_t)half;
        for (int i = 0; i < 7; i++) w = (w << bits) | (uint64_t)u[i];
        w = (w << (bits - 1)) | (uint64_t)(u[7] >> 1);
        for (int b = bits - 1; b >= 0; b--) { out[v * bits + b] = (uint8_t)(w & 0xFF); w >>= 8; }
    }
    return 0;
}

/* unpack_e8 (core/compact_storage.py:157-222), big-endian bytes. */
void lqo_unpack_e8(const uint8_t *in, int64_t n, int bits, float *q) {
    int64_t R = 1LL << (bits - 1);
    uint64_t cm = (1ULL << bits) - 1, um = (1ULL << (bits - 1)) - 1;
    for (int64_t v = 0; v < n; v++) {
        uint64_t w = 0;
        for (int b = 0; b < bits; b++) w = (w << 8) | in[v * bits + b];
        int64_t c7u = (int64_t)(w & um);
        w >>= (bits - 1);
        int64_t s[7], ps = 0;
        for (int i = 6; i >= 0; i--) { s[i] = (int64_t)(w & cm) - R; w >>= bits; }
        int coset = (int)(w & 1);
        for (int i = 0; i < 7; i++) ps += s[i];
        int64_t c7 = c7u * 2 + floormod2(ps) - R;
        float off = coset ? 0.5f : 0.f;
        for (int i = 0; i < 7; i++) q[8 * v + i] = (float)s[i] + off;
        q[8 * v + 7] = (float)c7 + off;
    }
}

/* ------------------------------------------------------------- argsort --- */

/* numpy.argsort(kind='quicksort') on an x86 host with AVX512_SKX dispatches to
 * x86-simd-sort, whose n <= 256 case is a bitonic network over 8-lane
 * registers padded with the type maximum.  Each comparator keeps its own
 * element on equal keys.  This restatement reproduces numpy's tie order for
 * n <= 256 (checked exhaustively against numpy in tests/test_oracle.py).
 * Returns -1 for n > 256 (numpy then runs a SIMD quicksort not restated here). */
static void cx(int64_t *k, int32_t *a, int p, int q) {   /* p < q: min -> p */
    if (k[p] > k[q]) {
        int64_t tk = k[p]; k[p] = k[q]; k[q] = tk;
        int32_t ta = a[p]; a[p] = a[q]; a[q] = ta;
    }
}

static void net_sort8(int64_t *k, int32_t *a) {
    static const int m[6] = {1, 3, 1, 7, 2, 1};
    for (int s = 0; s < 6; s++)
        for (int i = 0; i < 8; i++) { int j = i ^ m[s]; if (i < j) cx(k, a, i, j); }
}

static void net_merge8(int64_t *k, int32_t *a) {
    static const int m[3] = {4, 2, 1};
    for (int s = 0; s < 3; s++)
        for (int i = 0; i < 8; i++) { int j = i ^ m[s]; if (i < j) cx(k, a, i, j); }
}

int lqo_argsort(const int64_t *keys, int n, int64_t pad, int32_t *out) {
    if (n > 256) return -1;
    if (n <= 0) return 0;
    int nv = 1;
    while (nv * 8 < n) nv *= 2;
    int64_t k[256];
    int32_t a[256];
    for (int i = 0; i < nv * 8; i++) { k[i] = i < n ? keys[i] : pad; a[i] = i < n ? i : -1; }
    for (int v = 0; v < nv; v++) net_sort8(k + 8 * v, a + 8 * v);
    for (int per = 2; per <= nv; per *= 2) {
        for (int g = 0; g < nv / per; g++) {
            int off = g * per;
            /* mirror compare between register i and register per-1-i */
            for (int i = 0; i < per / 2; i++) {
                int r1 = off + i, r2 = off + per - 1 - i;
                for (int l = 0; l < 8; l++) cx(k, a, 8 * r1 + l, 8 * r2 + 7 - l);
            }
            /* register-level half cleaners */
            for (int num = per / 2; num >= 2; num /= 2)
                for (int j = 0; j < per; j += num)
                    for (int i = 0; i < num / 2; i++) {
                        int r1 = off + j + i, r2 = off + j + i + num / 2;
                        for (int l = 0; l < 8; l++) cx(k, a, 8 * r1 + l, 8 * r2 + l);
                    }
            for (int i = 0; i < per; i++) net_merge8(k + 8 * (off + i), a + 8 * (off + i));
        }
    }
    for (int i = 0; i < n; i++) out[i] = a[i];
    return 0;
}

/* ---------------------------------------------------------------- rANS --- */

/* build_rans_table normalisation (core/gpu_ans.py:62-90).  Returns 0; -1 for
 * n > 1024 (the reference loops forever there); -2 when a pass needs an argsort
 * of more than 256 keys (the Python side then runs the loop with numpy). */
int lqo_build_table(const int64_t *counts, int n, int32_t *freqs) {
    if (n <= 0) return -3;
    if (n > LQO_L) return -1;
    int64_t total = 0;
    for (int i = 0; i < n; i++) total += counts[i];
    for (int i = 0; i < n; i++) {
        if (total == 0) { freqs[i] = 1; continue; }
        double f = (double)counts[i] / (double)total * (double)LQO_L;
        int32_t t = (int32_t)f;                 /* astype(int32): truncation */
        freqs[i] = t < 1 ? 1 : t;
    }
    int64_t keys[LQO_L];
    int32_t order[LQO_L];
    for (;;) {
        int64_t sum = 0;
        for (int i = 0; i < n; i++) sum += freqs[i];
        if (sum == LQO_L) break;
        int64_t diff = LQO_L - sum;
        if (diff > 0) {
            for (int i = 0; i < n; i++) keys[i] = -counts[i];
            if (lqo_argsort(keys, n, INT64_MAX, order) != 0) return -2;
            for (int64_t j = 0; j < diff; j++) freqs[order[j % n]] += 1;
        } else {
            for (int i = 0; i < n; i++) keys[i] = -(int64_t)freqs[i];
            if (lqo_argsort(keys, n, INT32_MAX, order) != 0) return -2;
            for (int64_t j = 0; j < -diff; j++) {
                int idx = order[j % n];
                if (freqs[idx] > 1) freqs[idx] -= 1;
            }
        }
    }
    return 0;
}

/* cumfreqs + slot->index lookup (core/gpu_ans.py:88-95). */
void lqo_table_lookup(const int32_t *freqs, int n, int32_t *cum, int32_t *lookup) {
    cum[0] = 0;
    for (int i = 0; i < n; i++) cum[i + 1] = cum[i] + freqs[i];
    for (int s = 0; s < n; s++)
        for (int j = cum[s]; j < cum[s + 1]; j++) lookup[j] = s;
}

/* rans_encode (core/gpu_ans.py:105-139) over symbol INDICES into a table.
 * words must hold max_words; returns the number of words written
 * (n_words + 1, the last one zero) or -1 if max_words is too small. */
int64_t lqo_rans_encode(const int32_t *idx, int64_t n, const int32_t *freqs, const int32_t *cum,
                        uint32_t *words, int64_t max_words, int64_t *state_out, int64_t *nbits_out) {
    /* bits are produced in reverse; collect them, then lay them out LSB-first */
    int64_t cap = 10 * n + 16;
    uint8_t *bits = (uint8_t *)malloc((size_t)cap);
    if (!bits) return -1;
    int64_t nb = 0;
    uint32_t x = LQO_L;
    for (int64_t i = n - 1; i >= 0; i--) {
        uint32_t fs = (uint32_t)freqs[idx[i]], cf = (uint32_t)cum[idx[i]];
        while (x >= 2 * fs) { bits[nb++] = (uint8_t)(x & 1); x >>= 1; }
        x = LQO_L * (x / fs) + cf + (x % fs);
    }
    int64_t n_words = (nb + 31) / 32;
    if (n_words + 1 > max_words) { free(bits); return -1; }
    memset(words, 0, (size_t)(n_words + 1) * 4);
    for (int64_t i = 0; i < nb; i++) {
        uint32_t b = bits[nb - 1 - i];
        words[i / 32] |= b << (i % 32);
    }
    free(bits);
    *state_out = x;
    *nbits_out = nb;
    return n_words + 1;
}

/* rans_decode_cpu (core/gpu_ans.py:146-168), returns symbol indices. */
void lqo_rans_decode(const uint32_t *words, int64_t n_bits, int64_t state, const int32_t *freqs,
                     const int32_t *cum, const int32_t *lookup, int64_t n, int32_t *out) {
    uint32_t x = (uint32_t)state;
    int64_t bp = 0;
    for (int64_t i = 0; i < n; i++) {
        uint32_t slot = x & (LQO_L - 1);
        int32_t si = lookup[slot];
        out[i] = si;
        x = (uint32_t)freqs[si] * (x >> LQO_LOG2_L) + slot - (uint32_t)cum[si];
        while (x < LQO_L && bp < n_bits) {
            uint32_t bit = (words[bp / 32] >> (bp % 32)) & 1u;
            x = (x << 1) | bit;
            bp++;
        }
    }
}
