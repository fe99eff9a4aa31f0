// Table-driven rANS stream decoder shared by the chunk decoder and the
// decode-attention kernels.
//
// Stream format (reference core/gpu_ans.py:105-168): L = 1024 table slots,
// the state x lives in [L, 2L) between symbols, one step is
//   slot = x - L;  s = lookup[slot];  x = f_s * (x >> 10) + slot - cum_s;
//   while x < L: x = 2 x + next stream bit        (bits LSB-first in words)
// Because x >> 10 == 1 for every state in [L, 2L), the step depends on the
// slot only: x' = f_s + slot - cum_s lies in [f_s, 2 f_s), it needs
// k = 10 - floor(log2 x') renormalisation bits (0 when x' >= L), and the next
// slot is (x' << k) - L plus those k bits.  One LUT entry per slot holds the
// symbol and that successor rule, so a step is one LDS read and two
// dependent ALU ops.
#pragma once

#include "lq_device.h"

namespace lq {

// LUT entry of one (stream, slot):
//   [3:0]   k, the renormalisation bits of the step (0..10)
//   [5:4]   zero, so that a 6-bit shift count or a 5-bit field width read
//           from the entry is k itself
//   [15:6]  symbol index (alphabet value - lo, < 1024)
//   [17:16] zero
//   [31:18] row * L + (x' << k) - L: the next slot before the k new bits are
//           added, inside an LDS block of up to 16 stream LUTs of L entries in
//           which this stream's LUT is row `row`
__host__ __device__ inline uint32_t lut_entry(uint32_t sym, uint32_t xp, uint32_t row) {
    uint32_t k = 0;
    while ((xp << k) < (uint32_t)LQ_L) k++;
    const uint32_t next = row * (uint32_t)LQ_L + (xp << k) - (uint32_t)LQ_L;
    return k | (sym << 6) | (next << 18);
}

__device__ __forceinline__ uint32_t lut_sym(uint32_t e) { return (e >> 6) & 1023u; }
__device__ __forceinline__ uint32_t lut_next(uint32_t e) { return e >> 18; }

// A lane's bit buffer: the next unread stream bits, most significant first
// (words are bit-reversed on the way in), then a single 1 bit (the sentinel),
// then zeros.  The sentinel stands in for a count of valid bits: fewer than
// 32 bits are valid exactly when the low word is zero, and push() finds the
// free space below the valid bits from its position.
struct BitBuf {
    uint64_t buf;

    // Start at bit `off` (0..31) of word w: 32 - off valid bits.
    __device__ __forceinline__ void init(uint32_t w, uint32_t off) {
        buf = (((uint64_t)__builtin_bitreverse32(w) << 32) | 0x80000000u) << (off & 31u);
    }
    __device__ __forceinline__ bool low() const { return (uint32_t)buf == 0u; }
    // Append the 32 bits of word w below the valid ones; needs low().
    __device__ __forceinline__ void push(uint32_t w) {
        const uint32_t hi = (uint32_t)(buf >> 32);
        const uint32_t t = (uint32_t)__builtin_ctz(hi);   // sentinel bit of hi (hi != 0 when low())
        const uint64_t y = (((uint64_t)__builtin_bitreverse32(w) << 32) | 0x80000000u) >> (31u - t);
        // high word: (hi & (hi - 1)) | y_hi, i.e. the old sentinel cleared
        // (bitop3 truth table 0xEA: (S0 & S1) | S2)
        const uint32_t nhi = __builtin_amdgcn_bitop3_b32(hi, hi - 1u, (uint32_t)(y >> 32), 0xEA);
        buf = ((uint64_t)nhi << 32) | (uint32_t)y;
    }
    // Take the k bits of LUT entry e (at least k bits valid): their value,
    // first bit most significant.  They are the bits that a 64-bit shift by
    // k moves out of the high word (k = 0 moves none), so the value is one
    // shift of the high word, zero-extended, read directly by the entry.
    __device__ __forceinline__ uint32_t take(uint32_t e) {
        const uint32_t bits = (uint32_t)(((uint64_t)(uint32_t)(buf >> 32) << (e & 63u)) >> 32);
        buf <<= (e & 63u);
        return bits;
    }
};

// ---------------------------------------------------------------------------
// Block-phase decoding of one (stream, checkpoint block) task per lane.
//
// A workgroup holds the 8 coordinate streams of one coset for a run of
// blocks; lane (block b, coordinate idx) owns stream idx of block b.  The
// lane decodes in phases of 8 steps:
//   * its bitstream words reach the decoder through a 16-word ring in LDS
//     (column `tid` of ring[kRing][LANES]) that holds the stream's 16-byte
//     aligned 4-word groups; a top-up is one aligned 16-byte load, issued at
//     one phase boundary and written to the ring at the next, so the decode
//     steps never wait on global memory;
//   * each step stages the symbol index in LDS (row b of the staging, 8 u16
//     per step) and walks the block's coset bitmap (words already restricted
//     to the coset's vectors) to find the vector the 8 lanes just decoded;
//   * after the phase, lane idx owns the vector of step idx: its 8 symbol
//     indices are row idx of the staging and its block position is returned.
// Reads stay inside the aligned 16-byte groups that hold the block's words
// up to two words after its last bit (the stream needs 2 words of slack after
// its n_words + 1); such a group never crosses a page.
constexpr int kPhase = 8;    // decode steps per phase
constexpr int kRing = 16;    // bitstream words per lane in the LDS ring

template <int LANES>
struct PhaseLane {
    const uint32_t* gs;     // the 16-byte aligned group holding the block's first word
    uint32_t* rcol;         // this lane's ring column
    int glim;               // first word (group index * 4, from gs) of the last readable group
    int ld, rd;             // next word (from gs) to load into the ring / to move into pre
    BitBuf bb;
    uint32_t pre, e;
    uint4 q;
    bool inflight;
    const uint32_t* bmr;    // the block's coset bitmap row (kBlk / 32 + 1 words, last one zero)
    int wi;
    uint32_t wv, wn;

    __device__ __forceinline__ uint4 group(int i) const {   // i: a multiple of 4
        return *reinterpret_cast<const uint4*>(gs + (i < glim ? i : glim));
    }
    __device__ __forceinline__ void land(int i, const uint4& g) {   // ring slots i .. i + 3 (i % 4 == 0)
        uint32_t* p = rcol + (i & (kRing - 1)) * LANES;
        p[0] = g.x;
        p[LANES] = g.y;
        p[2 * LANES] = g.z;
        p[3 * LANES] = g.w;
    }

    // stream_words: the stream; bit_off / end_bit: the block's first bit and
    // the next block's first bit (or the stream's n_bits); state: checkpoint
    // state; lut: LDS LUT block, row: this stream's row in it.
    __device__ __forceinline__ void init(const uint32_t* stream_words, uint32_t bit_off, int64_t end_bit, uint32_t state,
                                         const uint32_t* lut, int row, uint32_t* ring_col, const uint32_t* bm_row) {
        const uint32_t* sw = stream_words + (bit_off >> 5);
        const int o = (int)((reinterpret_cast<uintptr_t>(sw) >> 2) & 3u);
        gs = sw - o;
        const int wlim = (int)((end_bit >> 5) + 2 - (int64_t)(bit_off >> 5));   // last readable word, from sw
        glim = (wlim + o) & ~3;
        rcol = ring_col;
        const uint4 g0 = group(0), g1 = group(4), g2 = group(8);
        land(0, g0);
        land(4, g1);
        land(8, g2);
        ld = 12;
        rd = o + 2;
        bb.init(rcol[o * LANES], bit_off);
        pre = rcol[(o + 1) * LANES];
        refill();
        e = lut[row * kL + (int)state - kL];
        inflight = false;
        bmr = bm_row;
        wi = 0;
        wv = bmr[0];
        wn = bmr[1];
    }

    __device__ __forceinline__ void refill() {
        if (bb.low()) {
            bb.push(pre);
            pre = rcol[(rd & (kRing - 1)) * LANES];
            rd++;
        }
    }

    // Phase boundary: land the previous top-up, issue the next one.  A phase
    // moves at most 3 words out of the ring and a top-up (4 words) is issued
    // only if it fits even when none is consumed, so every phase starts with
    // at least 3 words in the ring (at least 6 after init).
    __device__ __forceinline__ void boundary() {
        if (inflight) {
            land(ld, q);
            ld += 4;
            inflight = false;
        }
        if (ld - rd <= kRing - 4) {
            q = group(ld);
            inflight = true;
        }
    }

    // One decode step: stage the current symbol index at stg_j, find its
    // vector, move to the next symbol.  Returns the vector's block position.
    __device__ __forceinline__ int step(uint16_t* stg_j, const char* lutb) {
        *stg_j = (uint16_t)lut_sym(e);
        if (wv == 0) {
            wi++;
            wv = wn;
            wn = bmr[wi + 1 <= kBlk / 32 ? wi + 1 : kBlk / 32];
            while (wv == 0) {   // a word with no vector of this coset
                wi++;
                wv = wn;
                wn = bmr[wi + 1 <= kBlk / 32 ? wi + 1 : kBlk / 32];
            }
        }
        const int vl = (wi << 5) | __builtin_ctz(wv);
        wv &= wv - 1u;
        const uint32_t addr = (lut_next(e) + bb.take(e)) << 2;
        e = *reinterpret_cast<const uint32_t*>(lutb + addr);
        return vl;
    }

    // Steps of one phase (m <= kPhase of them); my_stg: this lane's column of
    // the block's staging (step j at my_stg[8 j]).  Returns the block position
    // of the vector of step idx (the one this lane rebuilds).
    __device__ __forceinline__ int phase(int m, int idx, uint16_t* my_stg, const char* lutb) {
        int vsv = 0;
        if (m == kPhase) {
#pragma unroll
            for (int j = 0; j < kPhase; j++) {
                if (j % 3 == 0) refill();
                const int vl = step(my_stg + 8 * j, lutb);
                vsv = idx == j ? vl : vsv;
            }
        } else {
#pragma unroll
            for (int j = 0; j < kPhase; j++) {
                if (j < m) {
                    if (j % 3 == 0) refill();
                    const int vl = step(my_stg + 8 * j, lutb);
                    vsv = idx == j ? vl : vsv;
                }
            }
        }
        return vsv;
    }
};

// ---------------------------------------------------------------------------
// Rank-staged decoding of one (stream, checkpoint block) task per lane, used
// by the whole-line chunk decoder.  Like PhaseLane, but:
//   * the ring holds 12 words (three aligned 4-word groups) in a per-wave
//     column-major layout (word slot s of lane l at rcol[s * 64]), so a
//     1024-lane workgroup fits its 16 LUTs, rings and staging in LDS;
//   * the lane does not track vector positions: step j of a phase stages its
//     symbol index at the caller's slot j, in coset-rank order, and the
//     caller maps block positions to ranks when it rebuilds vectors;
//   * phases are always 8 steps: steps past the lane's last symbol decode
//     garbage from in-bounds LDS and ring words, which the caller never reads.
// Ring invariant (top-ups of 4 words, at most 3 words moved into pre per
// phase): a top-up is issued only when the group it lands in is not the one
// being read (then at most 8 words are unread, so it overwrites no unread
// word), and every phase starts with at least 3 unread words.
constexpr int kLineRing = 12;

// A 32-bit LDS word pointer: arithmetic and compares on it stay 32-bit.
typedef __attribute__((address_space(3))) uint32_t lds_u32;

struct LineLane {
    const uint32_t* gs;     // the 16-byte aligned group holding the block's first word
    lds_u32* rcol;          // this lane's ring column (slot stride 64 words)
    int glim;               // first word (from gs) of the last readable group
    int ld;                 // next word (from gs) to load into the ring (multiple of 4)
    const lds_u32* rq;      // ring word to move into pre next
    lds_u32* lp;            // first ring word of the group the next top-up lands in
    BitBuf bb;
    uint32_t pre, e;
    uint4 q;
    bool inflight;

    __device__ __forceinline__ uint4 group(int i) const {   // i: a multiple of 4
        return *reinterpret_cast<const uint4*>(gs + (i < glim ? i : glim));
    }
    __device__ __forceinline__ static void land(lds_u32* p, const uint4& g) {   // the 4 ring slots from p
        p[0] = g.x;
        p[64] = g.y;
        p[128] = g.z;
        p[192] = g.w;
    }

    // As PhaseLane::init (without the bitmap row).
    __device__ __forceinline__ void init(const uint32_t* stream_words, uint32_t bit_off, int64_t end_bit, uint32_t state,
                                         const uint32_t* lut, int row, uint32_t* ring_col) {
        const uint32_t* sw = stream_words + (bit_off >> 5);
        const int o = (int)((reinterpret_cast<uintptr_t>(sw) >> 2) & 3u);
        gs = sw - o;
        const int wlim = (int)((end_bit >> 5) + 2 - (int64_t)(bit_off >> 5));   // last readable word, from sw
        glim = (wlim + o) & ~3;
        rcol = (lds_u32*)ring_col;
        const uint4 g0 = group(0), g1 = group(4), g2 = group(8);
        land(rcol, g0);
        land(rcol + 4 * 64, g1);
        land(rcol + 8 * 64, g2);
        ld = 12;
        lp = rcol;
        rq = rcol + (o + 2) * 64;
        bb.init(rcol[o * 64], bit_off);
        pre = rcol[(o + 1) * 64];
        refill();
        e = lut[row * kL + (int)state - kL];
        inflight = false;
    }

    __device__ __forceinline__ void refill() {
        if (bb.low()) {
            bb.push(pre);
            pre = *rq;
            rq = rq == rcol + (kLineRing - 1) * 64 ? rcol : rq + 64;
        }
    }

    // Phase boundary: land the previous top-up, issue the next one if the
    // lane still decodes (`more`) and the ring has room for it.
    __device__ __forceinline__ void boundary(bool more) {
        if (inflight) {
            land(lp, q);
            lp = lp == rcol + 8 * 64 ? rcol : lp + 4 * 64;
            inflight = false;
        }
        // rq lies in the landing group iff it is 0 .. 1023 bytes past lp
        const uint32_t qoff = (uint32_t)(uintptr_t)rq - (uint32_t)(uintptr_t)lp;
        if (more && qoff >= 4u * 64u * 4u) {
            q = group(ld);
            ld += 4;
            inflight = true;
        }
    }

    __device__ __forceinline__ void step(uint16_t* stg_j, const char* lutb) {
        *stg_j = (uint16_t)lut_sym(e);
        const uint32_t addr = (lut_next(e) + bb.take(e)) << 2;
        e = *reinterpret_cast<const uint32_t*>(lutb + addr);
    }

    // kPhase steps; step j stages at stg[8 j].
    __device__ __forceinline__ void phase(uint16_t* stg, const char* lutb) {
#pragma unroll
        for (int j = 0; j < kPhase; j++) {
            if (j % 3 == 0) refill();
            step(stg + 8 * j, lutb);
        }
    }
};

// c7 parity of a staged vector: parity of the seven free coordinates, i.e.
// of their indices and of the alphabet lows (lpar).
__device__ __forceinline__ uint32_t staged_parity(const uint4& r, uint32_t lpar) {
    const uint32_t px = r.x ^ r.y ^ r.z ^ (r.w & 0xffffu);
    return (px ^ (px >> 16) ^ lpar) & 1u;
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Two dequantised fp16 values (q + lo + off) * scale from a pair of 16-bit
// symbol indices (< 1024), in packed fp16 arithmetic.  (1024 + i) has the bit
// pattern 0x6400 | i in fp16, so OR + subtract gives i exactly; adding the
// half-integer lo + off is exact for |value| < 1024, and the product rounds
// once, to the fp16 nearest to the exact product, which is what rounding the
// (exact) fp32 product q * scale to fp16 gives.
__device__ __forceinline__ uint32_t deq_pair_f16(uint32_t idx2, half2_t lo_off, half2_t sc2) {
    const uint32_t b = idx2 | 0x64006400u;
    half2_t v = __builtin_bit_cast(half2_t, b);
    const half2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    v = (v - k1024) + lo_off;
    return __builtin_bit_cast(uint32_t, v * sc2);
}

// Staged vector r (8 symbol indices) dequantised to 8 fp16 values, packed in
// pairs, given its coset's packed (lo + off) pairs and alphabet-low parity.
__device__ __forceinline__ uint4 deq_staged_f16(const uint4& r, const half2_t lo2[4], uint32_t lpar, half2_t sc2) {
    const uint32_t par = staged_parity(r, lpar);
    const uint32_t w3 = (r.w & 0xffffu) | (((r.w >> 16) * 2u + par) << 16);   // c7 index doubled + parity
    uint4 o;
    o.x = deq_pair_f16(r.x, lo2[0], sc2);
    o.y = deq_pair_f16(r.y, lo2[1], sc2);
    o.z = deq_pair_f16(r.z, lo2[2], sc2);
    o.w = deq_pair_f16(w3, lo2[3], sc2);
    return o;
}

// Biased symbol fields of the chunk decoder's LUTs.  When every alphabet of a
// chunk lies in the ranges checked below, the LUT symbol field of coordinate
// streams 0..6 holds the coordinate value + 512 and that of stream 7 holds
// floor(c7 / 2) + 256, instead of the alphabet index.  Then a staged vector
// needs no per-coset constants: the biases are even (the parity of the seven
// free fields is that of c0..c6), 2 u7 + parity = c7 + 512, and every field
// u < 1024, so fp16 (1024 + u) - 1536 is the coordinate exactly.
__device__ __forceinline__ bool chunk_biased(const lq_table* T16) {
    bool ok = true;
#pragma unroll
    for (int st = 0; st < LQ_STREAMS; st++) {
        const int n = T16[st].n_sym, lo = T16[st].lo;
        const int lim = (st & 7) < 7 ? 512 : 256;
        ok = ok && (n == 0 || (lo >= -lim && lo + n - 1 < lim));
    }
    return ok;
}

// A staged vector of biased fields dequantised to 8 fp16 values, packed in
// pairs: ((1024 + u) - 1536 + off) * scale, exact up to the one rounding of
// the product (off = 0 or 1/2, |coordinate| <= 512).
__device__ __forceinline__ uint4 deq_biased_f16(const uint4& r, half2_t off2, half2_t sc2) {
    const uint32_t px = r.x ^ r.y ^ r.z ^ (r.w & 0xffffu);
    const uint32_t par = (px ^ (px >> 16)) & 1u;
    const uint32_t w3 = (r.w & 0xffffu) | (((r.w >> 16) * 2u + par) << 16);
    const half2_t k1536 = {(_Float16)1536.0f, (_Float16)1536.0f};
    const uint32_t in[4] = {r.x, r.y, r.z, w3};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        half2_t v = __builtin_bit_cast(half2_t, in[i] | 0x64006400u);
        v = (v - k1536) + off2;
        o[i] = __builtin_bit_cast(uint32_t, v * sc2);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// The lattice point of a staged vector of biased fields, in fp32 (exact).
__device__ __forceinline__ void lattice_biased_f32(const uint4& r, float off, float y[8]) {
    const uint32_t px = r.x ^ r.y ^ r.z ^ (r.w & 0xffffu);
    const int par = (int)((px ^ (px >> 16)) & 1u);
    const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int j = 0; j < 7; j++) {
        const int u = (int)((j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu));
        y[j] = (float)(u - 512) + off;
    }
    y[7] = (float)(2 * ((int)(r.w >> 16) - 256) + par) + off;
}

// Per-workgroup dequantisation constants of one coset of one chunk: the
// 8 alphabet lows, their parity, and the packed (lo + off) pairs; `small`
// says every value fits the packed fp16 path (alphabet within [-500, 500)).
struct CosetConsts {
    int lo[8];
    uint32_t lpar;
    half2_t lo2[4];
    float off;
    bool small;

    __device__ __forceinline__ void init(const lq_table* T, int c) {
        int losum = 0;
        small = true;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            lo[j] = T[j].lo;
            if (j < 7) losum += lo[j];
            small = small && lo[j] >= -500 && lo[j] + T[j].n_sym <= 500;
        }
        lpar = (uint32_t)losum & 1u;
        off = c ? 0.5f : 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float a = (float)lo[2 * j] + off;
            const float b = j < 3 ? (float)lo[2 * j + 1] + off : (float)(2 * lo[7]) + off;
            lo2[j] = half2_t{(_Float16)a, (_Float16)b};
        }
    }

    // The staged vector r (8 symbol indices) dequantised to 8 fp16 values,
    // packed in pairs; needs small.
    __device__ __forceinline__ uint4 deq_f16(const uint4& r, half2_t sc2) const {
        return deq_staged_f16(r, lo2, lpar, sc2);
    }

    // The per-coset constants of coset cp, picked per lane from the two cosets' sets.
    __device__ __forceinline__ void pick(bool cp, const CosetConsts& c0, const CosetConsts& c1) {
#pragma unroll
        for (int j = 0; j < 8; j++) lo[j] = cp ? c1.lo[j] : c0.lo[j];
        lpar = cp ? c1.lpar : c0.lpar;
        off = cp ? c1.off : c0.off;
#pragma unroll
        for (int j = 0; j < 4; j++)
            lo2[j] = __builtin_bit_cast(half2_t, cp ? __builtin_bit_cast(uint32_t, c1.lo2[j])
                                                    : __builtin_bit_cast(uint32_t, c0.lo2[j]));
        small = cp ? c1.small : c0.small;
    }

    // The same values in fp32 (exact products, before any fp16 rounding):
    // fma(index, scale, (lo + off) * scale).
    __device__ __forceinline__ void deq_f32(const uint4& r, float sc, float y[8]) const {
        const uint32_t par = staged_parity(r, lpar);
        const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t v = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
            if (j == 7) v = 2u * v + par;
            const float cst = ((float)(j < 7 ? lo[j] : 2 * lo[j]) + off) * sc;
            y[j] = __builtin_fmaf((float)v, sc, cst);
        }
    }
};

// Per-chunk escape constants, wave-uniform: the shift k_j of each coordinate
// and the first of its fine words.
struct EscCoords {
    int k[8];
    const uint32_t* w[8];
    __device__ __forceinline__ void init(const int32_t* ek, const int64_t* fo, const uint32_t* fine) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            k[j] = __builtin_amdgcn_readfirstlane(ek[j]);
            const int64_t o = fo[j];
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)o);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)o >> 32));
            w[j] = fine + (int64_t)(((uint64_t)hi << 32) | lo);
        }
    }
};

// A staged vector of an escaped chunk (coarse symbol fields in r) as its
// lattice point in fp32: coordinate j's coarse symbol is the field minus its
// bias (512, c8h 256) when the chunk's LUTs hold biased fields, else
// lo_j + index; the symbol is (coarse << k_j) plus its k_j raw low bits (bit
// v * k_j of the coordinate's fine words, least significant first), then
// c7 = 2 * c8h + (sum of the free symbols mod 2) (core/entropy_coder.py:71-89)
// and the coset offset.
__device__ __forceinline__ void lattice_escaped_f32(const uint4& r, const CosetConsts& cs, bool lut_biased,
                                                    const EscCoords& ec, int64_t v, float y[8]) {
    const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
    int sv[8];
    int par = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int idx = (int)((j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu));
        int val = lut_biased ? idx - (j < 7 ? 512 : 256) : cs.lo[j] + idx;
        const int k = ec.k[j];
        if (k) {
            const int64_t bit = v * k;
            const uint32_t* wp = ec.w[j] + (bit >> 5);
            const int sh = (int)(bit & 31);
            uint32_t f = wp[0] >> sh;
            if (sh + k > 32) f |= wp[1] << (32 - sh);
            val = val * (1 << k) + (int)(f & ((1u << k) - 1u));
        }
        sv[j] = val;
        if (j < 7) par += val;
    }
#pragma unroll
    for (int j = 0; j < 7; j++) y[j] = (float)sv[j] + cs.off;
    y[7] = (float)(2 * sv[7] + (par & 1)) + cs.off;
}

}  // namespace lq
