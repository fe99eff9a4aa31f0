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
//   [4:0]   31 - k          (shift that leaves the top k buffer bits in place)
//   [8:5]   k               (renormalisation bits, 0..10)
//   [18:9]  symbol index    (alphabet value - lo, < 1024)
//   [31:19] row * L + (x' << k) - L: the next slot before the k new bits are
//           added, inside an LDS block of up to 8 stream LUTs of L entries in
//           which this stream's LUT is row `row`
__host__ __device__ inline uint32_t lut_entry(uint32_t sym, uint32_t xp, uint32_t row) {
    uint32_t k = 0;
    while ((xp << k) < (uint32_t)LQ_L) k++;
    const uint32_t next = row * (uint32_t)LQ_L + (xp << k) - (uint32_t)LQ_L;
    return (31u - k) | (k << 5) | (sym << 9) | (next << 19);
}

__device__ __forceinline__ uint32_t lut_sym(uint32_t e) { return (e >> 9) & 1023u; }
__device__ __forceinline__ uint32_t lut_k(uint32_t e) { return (e >> 5) & 15u; }

// One lane's decoder of one stream from a checkpoint.
//
// buf holds the next unread stream bits, most significant first (words are
// bit-reversed on the way in), nbuf of them valid; pre is the next word.
// Loads never go past word (p >> 5) + 2 of the stream, p the first unread
// bit, so a stream needs two readable words after its n_words + 1.
struct StreamDec {
    const uint32_t* wp;   // next word to fetch into pre
    uint64_t buf;
    uint32_t nbuf, pre, e;

    // Start at stream bit `bit_off` with state `state` (in [L, 2L)); `lut` is
    // the LDS LUT block, `row` this stream's row in it.
    __device__ __forceinline__ void init(const uint32_t* stream_words, uint32_t bit_off, uint32_t state,
                                         const uint32_t* lut, int row) {
        const uint32_t* w = stream_words + (bit_off >> 5);
        buf = ((uint64_t)__builtin_bitreverse32(w[0]) << 32) << (bit_off & 31u);
        nbuf = 32u - (bit_off & 31u);
        pre = w[1];
        wp = w + 2;
        refill();
        e = lut[row * kL + (int)state - kL];
    }

    // Make at least 32 bits available (three steps' worth).
    __device__ __forceinline__ void refill() {
        if (nbuf < 32u) {
            buf |= (uint64_t)__builtin_bitreverse32(pre) << (32u - nbuf);
            nbuf += 32u;
            pre = *wp++;
        }
    }

    // Symbol index of the current symbol.
    __device__ __forceinline__ uint32_t sym() const { return lut_sym(e); }

    // Move to the next symbol: take the current symbol's k renormalisation
    // bits and look up the next slot.  Needs nbuf >= k (refill() every three
    // steps guarantees it).
    __device__ __forceinline__ void step(const uint32_t* lut) {
        const uint32_t bits = (uint32_t)(buf >> 33) >> (e & 31u);
        const uint32_t k = lut_k(e);
        const uint32_t slot = (e >> 19) + bits;
        buf <<= k;
        nbuf -= k;
        e = lut[slot];
    }
};

}  // namespace lq
