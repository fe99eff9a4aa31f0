// Resident (working) form of a compressed KV prefix and the decode-attention
// kernel that reads it, for gfx950.
//
// The rANS streams are the at-rest form of the cache (bit-exact with the
// reference).  A decode step cannot re-run rANS over a 32k-token prefix, so
// the cache also keeps the same lattice points in a fixed-width form: one
// b = 5 compact code word per vector (core/compact_storage.py:87-154), 40 bits
// split into a uint32 and a uint8 plane (layout in latticequant_amd.h), plus
// int16 exception entries for the rare vectors outside the 5-bit range.  A
// 16-token block of one kv head is 256 records stored group-major: record
// (slot, group) is vector 4*group + slot/16 of token slot%16 and sits at
// group * 64 + slot, so one group of a block is 64 records in a row.
//
// Decoding a record to fp16 is bit arithmetic: a 5-bit field u placed at bit
// 1 of a half whose high bits are 0x60 gives the fp16 number 512 + u +
// coset / 2 (the coset bit sits at bit 0; the spacing of fp16 numbers in
// [512, 1024) is 1/2), so one AND-OR turns two fields into a packed pair;
// subtracting 528 leaves c exactly (c the lattice coordinate, a multiple of
// 1/2), and a packed multiply by the token's fp16 scale s rounds the exact
// product once: fp16(c * s), the value _decompress_chunk writes, for every
// fp16 s (subnormal products included).  The MFMA operands are therefore
// the fp16 K / V the reference's attention reads.
//
// lq_resident_attention: per (kv head, split) one workgroup of eight waves; a
// wave takes 32-token tiles:
//   S = Q K^T        8 MFMA 16x16x32 (rows: the group's query heads, spread so
//                    that query head h sits in row 4 (h % 4) + h / 4); lane l
//                    decodes records (slot l, group c) of each block
//   online softmax   exp2, row max by DPP within 16 lanes; P (fp16) through
//                    LDS into the A operand layout
//   O += P V         lane l decodes vector l % 16 of 8 consecutive tokens, and
//                    MFMA mm's column n is dimension 8 n + mm, so the V pairs
//                    become B operands in registers (v_perm), without LDS
// then the waves merge their (m, l, O) in LDS, each workgroup writes one
// record per query head, and the last workgroup of a kv head (device-scope
// counter) merges the records and writes the output.
#include <climits>
#include <cmath>
#include <mutex>

#include "lq_device.h"

using namespace lq;

namespace {

inline int launch_status() { return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_LAUNCH; }

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kHd = 128;
constexpr int kRB = 16;                       // tokens per resident block
constexpr uint32_t kPairBias = 0x60206020u;   // fp16 pair (528, 528)
constexpr uint32_t kFieldMask = 0x003E003Eu;  // bits 1..5 of both halves
constexpr uint32_t kLsbMask = 0x08420842u;    // low bits of u0..u5 in the a word

__device__ __forceinline__ uint32_t unbias(uint32_t v) {
    const h2_t r = __builtin_bit_cast(h2_t, v) - __builtin_bit_cast(h2_t, kPairBias);
    return __builtin_bit_cast(uint32_t, r);
}

// One record -> four fp16 pairs 528 + c of coordinates (0,1) (2,3) (4,5) (6,7).
__device__ __forceinline__ void rec_pairs(uint32_t a, uint32_t b, uint32_t p[4]) {
    // (coset bit at bit 0 and 16) | 0x60006000: byte 0 of a copied to byte 2
    // by one byte permute, then one AND-OR (a select between two constants
    // would take three instructions)
    const uint32_t kc = (__builtin_amdgcn_perm(0u, a, 0x0c000c00u) & 0x00010001u) | 0x60006000u;
    p[0] = (a & kFieldMask) | kc;
    p[1] = ((a >> 5) & kFieldMask) | kc;
    p[2] = ((a >> 10) & kFieldMask) | kc;
    const uint32_t c7h = ((b >> 5) & 7u) | ((a >> 13) & 8u);
    const uint32_t par = ((uint32_t)__builtin_popcount(a & kLsbMask) + b) & 1u;
    const uint32_t u7 = (c7h << 1) | par;
    p[3] = kc | ((b & 31u) << 1) | (u7 << 17);
}

// Records of tokens t and t+1 (same vector) -> eight fp16 pairs
// (coordinate i of t, coordinate i of t+1), values 528 + c.
__device__ __forceinline__ void rec_pairs_tok(uint32_t a0, uint32_t b0, uint32_t a1, uint32_t b1, uint32_t p[8]) {
    const uint32_t lo = __builtin_amdgcn_perm(a1, a0, 0x05040100u);   // a0[15:0] | a1[15:0] << 16
    const uint32_t hi = __builtin_amdgcn_perm(a1, a0, 0x07060302u);   // a0[31:16] | a1[31:16] << 16
    const uint32_t kc = 0x60006000u | (lo & 0x00010001u);             // coset of t at bit 0, of t+1 at bit 16
    p[0] = (lo & kFieldMask) | kc;
    p[2] = ((lo >> 5) & kFieldMask) | kc;
    p[4] = ((lo >> 10) & kFieldMask) | kc;
    p[1] = (hi & kFieldMask) | kc;
    p[3] = ((hi >> 5) & kFieldMask) | kc;
    p[5] = ((hi >> 10) & kFieldMask) | kc;
    const uint32_t h0 = ((b0 >> 5) & 7u) | ((a0 >> 13) & 8u);
    const uint32_t h1 = ((b1 >> 5) & 7u) | ((a1 >> 13) & 8u);
    const uint32_t q0 = ((uint32_t)__builtin_popcount(a0 & kLsbMask) + b0) & 1u;
    const uint32_t q1 = ((uint32_t)__builtin_popcount(a1 & kLsbMask) + b1) & 1u;
    p[6] = kc | ((b0 & 31u) << 1) | ((b1 & 31u) << 17);
    p[7] = kc | (((h0 << 1) | q0) << 1) | (((h1 << 1) | q1) << 17);
}

// int16 lattice values 2c -> fp16 pair of the coordinates c (exact)
__device__ __forceinline__ uint32_t pair_from_i16(int a, int b) {
    const h2_t r = {(_Float16)((float)a * 0.5f), (_Float16)((float)b * 0.5f)};
    return __builtin_bit_cast(uint32_t, r);
}

// fp16 pairs of coordinates c times the packed fp16 scales m = (s_lo, s_hi):
// fp16(c * s), one rounding of the exact product
template <int N>
__device__ __forceinline__ void mul_pairs(uint32_t p[N], uint32_t m) {
#pragma unroll
    for (int i = 0; i < N; i++)
        p[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, p[i]) * __builtin_bit_cast(h2_t, m));
}

__device__ __forceinline__ h8_t as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint4 u = make_uint4(a, b, c, d);
    return __builtin_bit_cast(h8_t, u);
}

// ------------------------------------------------------------ producer --

// encode one lattice point (integer coordinates ic of the coset
// representative, coset bit cs) as a record; false when out of range
__device__ __forceinline__ bool rec_encode(const float ic[8], int cs, uint32_t* a, uint32_t* b) {
    int u[8];
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float f = ic[i] + 16.0f;
        ok = ok && f >= 0.0f && f <= 31.0f;
        u[i] = ok ? (int)f : 0;
    }
    if (!ok) { *a = 0u; *b = 0u; return false; }
    const uint32_t c7h = (uint32_t)u[7] >> 1;
    *a = (uint32_t)cs | ((uint32_t)u[0] << 1) | ((uint32_t)u[2] << 6) | ((uint32_t)u[4] << 11) |
         ((c7h >> 3) << 16) | ((uint32_t)u[1] << 17) | ((uint32_t)u[3] << 22) | ((uint32_t)u[5] << 27);
    *b = (uint32_t)u[6] | ((c7h & 7u) << 5);
    return true;
}

// lattice point of vector (head hh, token t, vector g) of x with IEEE x / s
__device__ __forceinline__ int res_point(const void* x, int dtype, int64_t T, int64_t hh, int64_t t, int g, float s,
                                         float ic[8]) {
    float xv[8], tv[8];
    load8(x, dtype, (hh * T + t) * (kHd / 8) + g, xv);
#pragma unroll
    for (int i = 0; i < 8; i++) tv[i] = xv[i] / s;
    return e8_nearest_fast(tv, ic);
}

// grid (t_tokens / 16, n_heads), 256 threads: wave = group, lane = slot
__global__ __launch_bounds__(256) void k_res_quant(const void* __restrict__ x, int dtype, int64_t T,
                                                   const float* __restrict__ scale32,
                                                   const uint16_t* __restrict__ scale16, lq_resident r, int64_t h0,
                                                   int64_t blk0, uint32_t* __restrict__ cnt) {
    __shared__ unsigned long long wm[4];
    const int tid = threadIdx.x, grp = tid >> 6, slot = tid & 63;
    const int64_t bb = blockIdx.x, hh = blockIdx.y;
    const int64_t t = bb * kRB + (slot & 15);
    const int g = 4 * grp + (slot >> 4);
    float ic[8];
    const int cs = res_point(x, dtype, T, hh, t, g, scale32[hh], ic);
    uint32_t a, b;
    const bool ok = rec_encode(ic, cs, &a, &b);
    const int64_t rb = (h0 + hh) * r.cap_blocks + blk0 + bb;
    r.a[rb * 256 + grp * 64 + slot] = a;
    r.b[rb * 256 + grp * 64 + slot] = (uint8_t)b;
    const unsigned long long m = __ballot(!ok);
    if (slot == 0) {
        r.mask[rb * 4 + grp] = m;
        wm[grp] = m;
    }
    if (grp == 0 && slot < kRB) r.scale[(h0 + hh) * r.cap_blocks * kRB + (blk0 + bb) * kRB + slot] = scale16[hh];
    __syncthreads();
    if (tid == 0) {
        // header: count and the first seven exceptions in (group, slot) order
        uint64_t hdr = 0;
        int n = 0;
        for (int c = 0; c < 4; c++) {
            unsigned long long mm = wm[c];
            while (mm) {
                const int sl = __ffsll((long long)mm) - 1;
                mm &= mm - 1ull;
                if (n < 7) hdr |= (uint64_t)(sl | (c << 6)) << (8 * (n + 1));
                n++;
            }
        }
        hdr |= (uint64_t)(n < 255 ? n : 255);
        r.meta[rb * 4 + 0] = (uint32_t)hdr;
        r.meta[rb * 4 + 1] = (uint32_t)(hdr >> 32);
        r.meta[rb * 4 + 3] = (uint32_t)n;
        cnt[hh * gridDim.x + bb] = (uint32_t)n;
    }
}

// exclusive scan of the per-block exception counts (one workgroup) -> base,
// starting at *n_exc, which advances by the total
__global__ __launch_bounds__(256) void k_res_scan(const uint32_t* __restrict__ cnt, int64_t nblk_call,
                                                  int64_t n_heads_call, lq_resident r, int64_t h0, int64_t blk0) {
    __shared__ uint32_t part[256];
    const int tid = threadIdx.x;
    const int64_t n = nblk_call * n_heads_call;
    const int64_t per = (n + 255) / 256;
    const int64_t lo = tid * per, hi = lo + per < n ? lo + per : n;
    uint32_t s = 0;
    for (int64_t i = lo; i < hi; i++) s += cnt[i];
    part[tid] = s;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const uint32_t v = tid >= off ? part[tid - off] : 0u;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    const uint32_t start = (uint32_t)*r.n_exc;
    uint32_t run = start + (tid ? part[tid - 1] : 0u);
    for (int64_t i = lo; i < hi; i++) {
        const int64_t hh = i / nblk_call, bb = i % nblk_call;
        r.meta[((h0 + hh) * r.cap_blocks + blk0 + bb) * 4 + 2] = run;
        run += cnt[i];
    }
    __syncthreads();
    if (tid == 255) *r.n_exc = (int32_t)(start + part[255]);
}

// exception entries: the vectors flagged by k_res_quant, recomputed
__global__ __launch_bounds__(256) void k_res_fill(const void* __restrict__ x, int dtype, int64_t T,
                                                  const float* __restrict__ scale32, lq_resident r, int64_t h0,
                                                  int64_t blk0) {
    const int tid = threadIdx.x, grp = tid >> 6, slot = tid & 63;
    const int64_t bb = blockIdx.x, hh = blockIdx.y;
    const int64_t rb = (h0 + hh) * r.cap_blocks + blk0 + bb;
    const unsigned long long m0 = r.mask[rb * 4 + 0], m1 = r.mask[rb * 4 + 1], m2 = r.mask[rb * 4 + 2],
                             m3 = r.mask[rb * 4 + 3];
    if ((m0 | m1 | m2 | m3) == 0ull) return;
    const unsigned long long m = grp == 0 ? m0 : grp == 1 ? m1 : grp == 2 ? m2 : m3;
    if (!((m >> slot) & 1ull)) return;
    int before = 0;
    if (grp > 0) before += __popcll(m0);
    if (grp > 1) before += __popcll(m1);
    if (grp > 2) before += __popcll(m2);
    before += __popcll(m & ((1ull << slot) - 1ull));
    const int64_t idx = (int64_t)r.meta[rb * 4 + 2] + before;
    if (idx >= r.exc_cap) {
        atomicOr(r.status, LQ_RES_ST_EXC_OVERFLOW);
        return;
    }
    float ic[8];
    const int cs = res_point(x, dtype, T, hh, bb * kRB + (slot & 15), 4 * grp + (slot >> 4), scale32[hh], ic);
    int16_t e[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float v = fminf(fmaxf(2.0f * ic[i] + (float)cs, -32768.0f), 32767.0f);
        e[i] = (int16_t)v;
    }
    uint4 w;
    w.x = (uint16_t)e[0] | ((uint32_t)(uint16_t)e[1] << 16);
    w.y = (uint16_t)e[2] | ((uint32_t)(uint16_t)e[3] << 16);
    w.z = (uint16_t)e[4] | ((uint32_t)(uint16_t)e[5] << 16);
    w.w = (uint16_t)e[6] | ((uint32_t)(uint16_t)e[7] << 16);
    reinterpret_cast<uint4*>(r.exc)[idx] = w;
}

// exception entry idx -> 8 lattice values 2c
__device__ __forceinline__ void exc_load(const int16_t* exc, int64_t idx, int v[8]) {
    const uint4 w = reinterpret_cast<const uint4*>(exc)[idx];
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = (int)(int16_t)(ww[i] & 0xffffu);
        v[2 * i + 1] = (int)(int16_t)(ww[i] >> 16);
    }
}

// grid (n_blocks, n_heads), 256 threads: one record per thread
__global__ __launch_bounds__(256) void k_res_dequant(lq_resident r, int64_t h0, int64_t blk0, int64_t nblk_call,
                                                     void* __restrict__ out, int out_dtype) {
    const int tid = threadIdx.x, grp = tid >> 6, slot = tid & 63;
    const int64_t bb = blockIdx.x, hh = blockIdx.y;
    const int64_t rb = (h0 + hh) * r.cap_blocks + blk0 + bb;
    const int64_t tok = bb * kRB + (slot & 15);
    const int g = 4 * grp + (slot >> 4);
    const unsigned long long m = r.mask[rb * 4 + grp];
    int v2[8];
    if ((m >> slot) & 1ull) {
        int before = 0;
        for (int c = 0; c < grp; c++) before += __popcll(r.mask[rb * 4 + c]);
        before += __popcll(m & ((1ull << slot) - 1ull));
        const int64_t idx = (int64_t)r.meta[rb * 4 + 2] + before;
        if (idx < r.exc_cap) {
            exc_load(r.exc, idx, v2);
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v2[i] = 0;
        }
    } else {
        uint32_t p[4];
        rec_pairs(r.a[rb * 256 + grp * 64 + slot], r.b[rb * 256 + grp * 64 + slot], p);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const h2_t h = __builtin_bit_cast(h2_t, p[i]);
            v2[2 * i] = (int)((float)h[0] * 2.0f) - 1056;   // 2 (528 + c) - 1056 = 2 c
            v2[2 * i + 1] = (int)((float)h[1] * 2.0f) - 1056;
        }
    }
    const float s = h2f(r.scale[(h0 + hh) * r.cap_blocks * kRB + (blk0 + bb) * kRB + (slot & 15)]);
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = ((float)v2[i] * 0.5f) * s;
    store8(out, out_dtype, (hh * nblk_call * kRB + tok) * (kHd / 8) + g, y);
}

// ----------------------------------------------------------- attention --

constexpr int kAW = 8;                          // waves per workgroup
constexpr int kTile = 32;                       // tokens per tile (two blocks)
constexpr int kWaveTiles = 4;
constexpr int kPtRow = 20;                      // uint32 per LDS P row (32 tokens fp16 + 16 B pad)
constexpr int kRecF = 4 + kHd;                  // floats per split record (m, l, 2 pad, o[128])
constexpr int kMaxRec = 2048;                   // (split, head) records one merge can take
constexpr int kMergeF = 4 * kMaxRec;            // floats of the merge buffer (3 record arrays + partial sums)
constexpr int kMergeH = kMergeF / (kAW * kHd);  // query heads per round of the workgroup merge
constexpr int kCtrStride = 64;                  // uint32 per completion counter (one per 256-byte line)

struct AttnArgs {
    lq_resident k, v;
    int64_t t_prefix, t_tail;
    const uint16_t* q;
    const uint16_t* tail_k;
    const uint16_t* tail_v;
    int group, nsp;
    float* rec;
    uint32_t* counter;
    uint16_t* out;
};

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// max / sum over the 16 lanes of a DPP row
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp<0x4E>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp<0x141>(v));   // row_half_mirror
    v = fmaxf(v, dpp<0x140>(v));   // row_mirror
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return v;
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- prefix tiles
//
// K lane layout (B operand of S = Q K^T): block x (0, 1), slot = lane: token
// 16 x + lane % 16, vectors 4 c + lane / 16 = records (slot lane, group c).
// V lane layout (B operand of O += P V): column n = lane % 16, token octet
// k8 = lane / 16 (tokens 8 k8 .. 8 k8 + 7 of the tile, block k8 / 2): the
// lane decodes the 8 records of vector n of those tokens (8 consecutive slots
// of group n / 4), and MFMA mm of P V takes dimension 8 n + mm of each token
// for column n, so the output column n of MFMA mm is dimension 8 n + mm and
// the decoded records feed the MFMAs without a transpose through LDS.
struct TileRaw {
    uint32_t ka[2][4];      // K record words of blocks 0, 1, groups 0..3
    uint32_t kb[2][4];      // their low bytes
    uint32_t ks[2];         // fp16 scale of the lane's K token of block 0, 1 (kept apart: combining
                            // them at load time would wait for every load in flight)
    uint4 va0, va1;         // V records of the lane's 8 tokens (vector lane % 16)
    uint2 vb;               // their low bytes
    uint4 vs;               // fp16 scales of those 8 tokens
    uint4 meta;             // lanes 0..3: block metadata of K block 0, 1, V block 0, 1
};

// a block's exception header and base from the tile's meta registers
// (i = 0, 1: K blocks, 2, 3: V blocks); wave-uniform
__device__ __forceinline__ uint64_t meta_hdr(const TileRaw& d, int i) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)d.meta.x, i);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)d.meta.y, i);
    return (uint64_t)lo | ((uint64_t)hi << 32);
}
__device__ __forceinline__ uint32_t meta_base(const TileRaw& d, int i) {
    return (uint32_t)__builtin_amdgcn_readlane((int)d.meta.z, i);
}

__device__ __forceinline__ void tile_load(const AttnArgs& A, int64_t kvh, int64_t t0, int64_t T, int lane,
                                          TileRaw& d) {
    // Blocks past the prefix (only block 1 of the last tile, T being a
    // multiple of 16) read the last block instead: every address is valid and
    // no branch waits on the loads; their tokens are masked out of the scores
    // and carry p = 0 into P V.  Every address is a wave-uniform base (scalar
    // registers) plus a per-lane 32-bit offset.
    const int64_t hb = kvh * A.k.cap_blocks;
    const int64_t last = T - kRB;
    const int64_t tb0 = min(t0, last), tb1 = min(t0 + 16, last);   // first tokens of the tile's blocks
    const int64_t rb0 = hb + tb0 / kRB;
    const uint32_t dblk = (uint32_t)(tb1 - tb0) / kRB;                // 1, or 0 when block 1 is clamped
#pragma unroll
    for (int x = 0; x < 2; x++) {
        const int64_t rb = x ? rb0 + dblk : rb0;
        const uint32_t* ka = A.k.a + rb * 256;
        const uint8_t* kb = A.k.b + rb * 256;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            d.ka[x][c] = ka[(uint32_t)(c * 64 + lane)];
            d.kb[x][c] = kb[(uint32_t)(c * 64 + lane)];
        }
        d.ks[x] = (A.k.scale + hb * kRB + (x ? tb1 : tb0))[(uint32_t)(lane & 15)];
    }
    {   // lanes 0..3 (and their copies): meta of K block 0, 1 and V block 0, 1.
        // A per-lane address keeps this a vector load: scalar loads share the
        // LDS wait counter and would stall every tile's LDS traffic.
        const int i = lane & 3;
        const uint32_t* mp = ((i & 2) ? A.v.meta : A.k.meta) + rb0 * 4;
        d.meta = *reinterpret_cast<const uint4*>(mp + (i & 1) * dblk * 4);
    }
    const int n = lane & 15, k8 = lane >> 4;
    // records of vector n of tokens 8 k8 .. 8 k8 + 7: block k8 / 2 of the tile
    const uint32_t r0 = (uint32_t)((k8 >> 1) * dblk * 256 + (n >> 2) * 64 + 16 * (n & 3) + 8 * (k8 & 1));
    const uint4* ap = reinterpret_cast<const uint4*>(A.v.a + rb0 * 256 + r0);
    d.va0 = ap[0];
    d.va1 = ap[1];
    d.vb = *reinterpret_cast<const uint2*>(A.v.b + rb0 * 256 + r0);
    d.vs = *reinterpret_cast<const uint4*>(A.v.scale + hb * kRB + tb0 + (uint32_t)((k8 >> 1) * dblk * 16 + 8 * (k8 & 1)));
}

// exception k of a block (0 <= k < count): slot | group << 6 from the header,
// or, past the header's seven entries, from the block's masks; -1 past the end
__device__ __forceinline__ int exc_code(const lq_resident& r, int64_t rb, uint64_t hdr, int k) {
    if (k < 7) return (int)((hdr >> (8 * (k + 1))) & 0xffu);
    int before = 0;
    for (int c = 0; c < 4; c++) {
        unsigned long long m = r.mask[rb * 4 + c];
        const int pc = __popcll(m);
        if (k < before + pc) {
            for (int q = before; q < k; q++) m &= m - 1ull;
            return (__ffsll((long long)m) - 1) | (c << 6);
        }
        before += pc;
    }
    return -1;
}

// Scores of block x: s += q . k over the four record groups, each group's K
// operand decoded (and, rarely, patched with exception entries) just before
// its MFMA, so that only one group's pairs are live at a time.
__device__ __forceinline__ void tile_k(const AttnArgs& A, const TileRaw& d, int64_t rb, int x, int lane,
                                       const h8_t qa[4], f4_t& s) {
    const uint64_t hdr = meta_hdr(d, x);
    const int n = (int)(hdr & 0xffu);
    const uint32_t mk = d.ks[x] * 0x00010001u;   // (s, s) of the lane's token
#pragma unroll
    for (int c = 0; c < 4; c++) {
        uint32_t p[4];
        rec_pairs(d.ka[x][c], d.kb[x][c], p);
#pragma unroll
        for (int i = 0; i < 4; i++) p[i] = unbias(p[i]);
        if (n) {   // rare: exception entries of group c replace records (uniform loop)
            const int64_t base = meta_base(d, x);
            const int cnt = n < 255 ? n : 4 * 64;
            for (int e = 0; e < cnt; e++) {
                const int code = exc_code(A.k, rb, hdr, e);
                if (code < 0) break;
                const int64_t idx = base + e;
                if ((code >> 6) == c && (code & 63) == lane && idx < A.k.exc_cap) {
                    int v[8];
                    exc_load(A.k.exc, idx, v);
#pragma unroll
                    for (int i = 0; i < 4; i++) p[i] = pair_from_i16(v[2 * i], v[2 * i + 1]);
                }
            }
        }
        mul_pairs<4>(p, mk);
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], as_h8(p[0], p[1], p[2], p[3]), s, 0, 0, 0);
    }
}

// V of the lane's 8 tokens (vector lane % 16), two tokens at a time:
// vp[k][i] = fp16 pair (dimension 8 n + i of token 2 k, of token 2 k + 1),
// dequantised -- the operand halves of P V's MFMA i as they are.
__device__ __forceinline__ void tile_v(const AttnArgs& A, const TileRaw& d, int64_t rb0, int lane,
                                       uint32_t vp[4][8]) {
    const int n = lane & 15, k8 = lane >> 4, xb = k8 >> 1;
    const uint32_t aw[8] = {d.va0.x, d.va0.y, d.va0.z, d.va0.w, d.va1.x, d.va1.y, d.va1.z, d.va1.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t bw = k < 2 ? d.vb.x : d.vb.y;
        rec_pairs_tok(aw[2 * k], bw >> (16 * (k & 1)), aw[2 * k + 1], bw >> (16 * (k & 1) + 8), vp[k]);
#pragma unroll
        for (int i = 0; i < 8; i++) vp[k][i] = unbias(vp[k][i]);
    }
    const uint64_t h0 = meta_hdr(d, 2), h1 = meta_hdr(d, 3);
    if ((h0 | h1) & 0xffull) {   // rare: exception entries replace records (uniform loops)
#pragma unroll 1
        for (int x = 0; x < 2; x++) {
            const uint64_t hdr = x ? h1 : h0;
            const int64_t base = x ? meta_base(d, 3) : meta_base(d, 2);
            const int cnt0 = (int)(hdr & 0xffu);
            const int cnt = cnt0 < 255 ? cnt0 : 4 * 64;
            for (int e = 0; e < cnt; e++) {
                const int code = exc_code(A.v, rb0 + x, hdr, e);
                if (code < 0) break;
                const int sl = code & 63, g = code >> 6;
                const int64_t idx = base + e;
                // the lane holding (slot sl, group g) of block x, and its token q
                const bool mine = xb == x && n == 4 * g + (sl >> 4) && (k8 & 1) == ((sl & 15) >> 3);
                if (mine && idx < A.v.exc_cap) {
                    int v[8];
                    exc_load(A.v.exc, idx, v);
                    const int q = sl & 7;
#pragma unroll
                    for (int k = 0; k < 4; k++)
#pragma unroll
                        for (int i = 0; i < 8; i++) {
                            h2_t h = __builtin_bit_cast(h2_t, vp[k][i]);
                            if (q == 2 * k) h[0] = (_Float16)((float)v[i] * 0.5f);
                            if (q == 2 * k + 1) h[1] = (_Float16)((float)v[i] * 0.5f);
                            vp[k][i] = __builtin_bit_cast(uint32_t, h);
                        }
                }
            }
        }
    }
    const uint32_t sw[4] = {d.vs.x, d.vs.y, d.vs.z, d.vs.w};   // scales of tokens (2 k, 2 k + 1)
#pragma unroll
    for (int k = 0; k < 4; k++) mul_pairs<8>(vp[k], sw[k]);
}

// ---- tail tiles (fp16 K / V, t_tail tokens, no prefetch)
__device__ __forceinline__ void tail_k(const AttnArgs& A, int64_t kvh, int64_t tb, int64_t T, int lane, h8_t kb[4]) {
    const int64_t t = tb + (lane & 15);
#pragma unroll
    for (int c = 0; c < 4; c++) {
        uint4 w = make_uint4(0u, 0u, 0u, 0u);
        if (t < T) w = *reinterpret_cast<const uint4*>(A.tail_k + (kvh * T + t) * kHd + 32 * c + 8 * (lane >> 4));
        kb[c] = __builtin_bit_cast(h8_t, w);
    }
}

__device__ __forceinline__ void tail_v(const AttnArgs& A, int64_t kvh, int64_t t0, int64_t T, int lane,
                                       uint32_t vp[4][8]) {
    const int n = lane & 15, k8 = lane >> 4;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int64_t t = t0 + 8 * k8 + 2 * k;
        uint4 w0 = make_uint4(0u, 0u, 0u, 0u), w1 = w0;
        if (t < T) w0 = *reinterpret_cast<const uint4*>(A.tail_v + (kvh * T + t) * kHd + 8 * n);
        if (t + 1 < T) w1 = *reinterpret_cast<const uint4*>(A.tail_v + (kvh * T + t + 1) * kHd + 8 * n);
        const uint32_t x0[4] = {w0.x, w0.y, w0.z, w0.w}, x1[4] = {w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            vp[k][2 * i] = __builtin_amdgcn_perm(x1[i], x0[i], 0x05040100u);
            vp[k][2 * i + 1] = __builtin_amdgcn_perm(x1[i], x0[i], 0x07060302u);
        }
    }
}

// Online softmax of one tile's scores, P through LDS into the A operand,
// O += P V with the B operand of MFMA mm = the lane's 8 tokens' dimension
// 8 n + mm, i.e. vp[0..3][mm].
template <int HPL>
__device__ __forceinline__ void tile_softmax_pv(int G, const f4_t s[2], const bool valid[2], int lane,
                                                const uint32_t vp[4][8], uint32_t* pt, float m_run[HPL],
                                                float l_run[HPL], f4_t o[8]) {
    const float c0 = 1.4426950408889634f / 11.313708498984761f;   // log2(e) / sqrt(128)
    _Float16* ph = reinterpret_cast<_Float16*>(pt);
#pragma unroll
    for (int i = 0; i < HPL; i++) {
        const int h = (lane >> 4) + 4 * i;
        const float z0 = valid[0] ? s[0][i] * c0 : -INFINITY;
        const float z1 = valid[1] ? s[1][i] * c0 : -INFINITY;
        const float mn = fmaxf(m_run[i], row16_max(fmaxf(z0, z1)));
        const float al = __builtin_amdgcn_exp2f(m_run[i] - mn);
        const float p0 = __builtin_amdgcn_exp2f(z0 - mn), p1 = __builtin_amdgcn_exp2f(z1 - mn);
        l_run[i] = l_run[i] * al + (p0 + p1);
        m_run[i] = mn;
#pragma unroll
        for (int mm = 0; mm < 8; mm++) o[mm][i] *= al;
        const bool hv = h < G;
        const int row = 4 * (lane >> 4) + i;
        ph[row * (2 * kPtRow) + (lane & 15)] = hv ? (_Float16)p0 : (_Float16)0.f;
        ph[row * (2 * kPtRow) + 16 + (lane & 15)] = hv ? (_Float16)p1 : (_Float16)0.f;
    }
    wave_lds_sync();
    // A = P rows (query heads) x 32 tokens, B = V 32 tokens x 16 columns
    const uint4 pa = *reinterpret_cast<const uint4*>(pt + (lane & 15) * kPtRow + 4 * (lane >> 4));
    const h8_t pA = __builtin_bit_cast(h8_t, pa);
#pragma unroll
    for (int mm = 0; mm < 8; mm++)
        o[mm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pA, as_h8(vp[0][mm], vp[1][mm], vp[2][mm], vp[3][mm]), o[mm], 0, 0, 0);
    wave_lds_sync();
}

// Decode of one prefix tile from its registers (rb0: resident block of the
// tile's first token): the scores s of its two blocks and the V pairs.
__device__ __forceinline__ void prefix_decode(const AttnArgs& A, const TileRaw& d, int64_t rb0, int64_t t0, int64_t T,
                                              int lane, const h8_t qa[4], f4_t s[2], bool valid[2],
                                              uint32_t vp[4][8]) {
#pragma unroll
    for (int x = 0; x < 2; x++) {
        s[x] = f4_t{0.f, 0.f, 0.f, 0.f};
        valid[x] = t0 + 16 * x + (lane & 15) < T;
        if (t0 + 16 * x < T)   // wave-uniform
            tile_k(A, d, rb0 + x, x, lane, qa, s[x]);
    }
    tile_v(A, d, rb0, lane, vp);
}

// The tail tiles this wave owns: tail tile tt goes to the kv head's wave
// (tt * W) / ntt, so the tiles spread over all splits instead of piling onto
// the first waves.  Each is taken before the wave's prefix tiles (their loads
// overlap the first prefix tile's), its K and V loads issued together.
template <int HPL>
__device__ __forceinline__ void tail_owned(const AttnArgs& A, int64_t kvh, int64_t gw, int64_t W, int64_t T, int lane,
                                           const h8_t qa[4], uint32_t* pt, float m_run[HPL], float l_run[HPL],
                                           f4_t o[8]) {
    const int64_t ntt = (T + kTile - 1) / kTile;
    const int64_t t_begin = (gw * ntt + W - 1) / W, t_end = ((gw + 1) * ntt + W - 1) / W;
    for (int64_t tt = t_begin; tt < t_end; tt++) {
        const int64_t t0 = tt * kTile;
        h8_t kb[2][4];
        uint32_t vp[4][8];
#pragma unroll
        for (int x = 0; x < 2; x++) tail_k(A, kvh, t0 + 16 * x, T, lane, kb[x]);
        tail_v(A, kvh, t0, T, lane, vp);
        f4_t s[2];
        bool valid[2];
#pragma unroll
        for (int x = 0; x < 2; x++) {
            s[x] = f4_t{0.f, 0.f, 0.f, 0.f};
            valid[x] = t0 + 16 * x + (lane & 15) < T;
#pragma unroll
            for (int c = 0; c < 4; c++) s[x] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], kb[x][c], s[x], 0, 0, 0);
        }
        tile_softmax_pv<HPL>(A.group, s, valid, lane, vp, pt, m_run, l_run, o);
    }
}

// The wave's prefix tiles.  The workgroup's tiles are the slots j of its
// round-robin share (wave w of split sp statically owns tiles sp * kAW + w +
// k * W): each wave starts with slot w, then takes the next free slot from a
// workgroup counter in LDS, so the waves of a workgroup finish together
// however their loads are delayed.  One register set: a tile's records are
// decoded (scores, V pairs) and the set is reloaded with the next tile's
// records, which are in flight during this tile's softmax and P V (a second
// set, loading a whole tile ahead, measured no faster).
template <int HPL>
__device__ __forceinline__ void prefix_tiles(const AttnArgs& A, int64_t kvh, int sp, int wave, int64_t W, int64_t T,
                                             int lane, const h8_t qa[4], uint32_t* pt, float m_run[HPL],
                                             float l_run[HPL], f4_t o[8], int* s_next) {
    const int64_t npt = (T + kTile - 1) / kTile;
    const int64_t gw = (int64_t)sp * kAW + wave;
    auto tile_of = [&](int j) -> int64_t { return (int64_t)sp * kAW + (j % kAW) + (int64_t)(j / kAW) * W; };
    int64_t g = tile_of(wave);
    if (g >= npt) {
        if (A.t_tail > 0) tail_owned<HPL>(A, kvh, gw, W, A.t_tail, lane, qa, pt, m_run, l_run, o);
        return;
    }
    const int64_t hb = kvh * A.k.cap_blocks;
    TileRaw d;
    tile_load(A, kvh, g * kTile, T, lane, d);
    if (A.t_tail > 0) tail_owned<HPL>(A, kvh, gw, W, A.t_tail, lane, qa, pt, m_run, l_run, o);
    while (true) {
        int jn = 0;
        if (lane == 0) jn = atomicAdd(s_next, 1);
        jn = __builtin_amdgcn_readfirstlane(jn) + kAW;
        const int64_t gn = tile_of(jn);
        const int64_t ta = g * kTile;
        f4_t s[2];
        bool valid[2];
        uint32_t vp[4][8];
        prefix_decode(A, d, hb + ta / kRB, ta, T, lane, qa, s, valid, vp);
        // Every use of this tile's registers is scheduled before the reload, and
        // the reload is unconditional (past the prefix it re-reads this tile,
        // from cache), so the next tile's loads land in place and nothing
        // waits on them before the next decode.
        __builtin_amdgcn_sched_barrier(0);
        tile_load(A, kvh, (gn < npt ? gn : g) * kTile, T, lane, d);
        tile_softmax_pv<HPL>(A.group, s, valid, lane, vp, pt, m_run, l_run, o);
        if (gn >= npt) break;
        g = gn;
    }
}

template <int HPL>
__global__ __launch_bounds__(kAW * 64) void k_res_attn(AttnArgs A) {
    __shared__ __align__(16) uint32_t s_pt[kAW][16 * kPtRow];
    __shared__ __align__(16) float s_buf[kMergeF];   // the waves' O rows, then the last workgroup's merge
    __shared__ float s_m[kAW][16], s_l[kAW][16];
    __shared__ float s_L[16];
    __shared__ int s_last, s_next;
    // the wave index is made wave-uniform explicitly so that all tile control
    // flow stays scalar (no exec-masked paths around in-flight loads)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = A.group;
    // one split = kAW waves; the kv head's waves share its prefix tiles and
    // then its tail tiles round-robin
    const int nsp = A.nsp;
    const int64_t kvh = (int64_t)blockIdx.x / nsp;
    const int sp = (int)((int64_t)blockIdx.x % nsp);
    const int64_t gw = (int64_t)sp * kAW + wave, W = (int64_t)nsp * kAW;

    // Q fragments: row m of the A operand is query head 4 (m % 4) + m / 4
    h8_t qa[4];
    {
        const int m = lane & 15, h = 4 * (m & 3) + (m >> 2);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            uint4 w = make_uint4(0u, 0u, 0u, 0u);
            if (h < G) w = *reinterpret_cast<const uint4*>(A.q + (kvh * G + h) * kHd + 32 * c + 8 * (lane >> 4));
            qa[c] = __builtin_bit_cast(h8_t, w);
        }
    }
    uint32_t* pt = s_pt[wave];
    for (int i = lane; i < 16 * kPtRow; i += 64) pt[i] = 0u;
    if (tid == 0) s_next = 0;
    __syncthreads();
    float m_run[HPL], l_run[HPL];
    f4_t o[8];
#pragma unroll
    for (int i = 0; i < HPL; i++) { m_run[i] = -INFINITY; l_run[i] = 0.f; }
#pragma unroll
    for (int mm = 0; mm < 8; mm++) o[mm] = f4_t{0.f, 0.f, 0.f, 0.f};
    if (A.t_prefix > 0) prefix_tiles<HPL>(A, kvh, sp, wave, W, A.t_prefix, lane, qa, pt, m_run, l_run, o, &s_next);
    else tail_owned<HPL>(A, kvh, gw, W, A.t_tail, lane, qa, pt, m_run, l_run, o);

    // ---- merge the waves' (m, l, O) in LDS, kMergeH query heads per round;
    // lane column n of MFMA mm holds dimension 8 n + mm of its rows
    float lsum[HPL];
#pragma unroll
    for (int i = 0; i < HPL; i++) lsum[i] = row16_sum(l_run[i]);
    // Records cross workgroups (and the XCDs' separate L2s): they are written
    // with device-scope stores (written through to the coherent level), which
    // complete before the counter increment, and read back with device-scope
    // loads.  No device-wide fence (an L2 write-back per workgroup) is needed.
    float* rec = A.rec + ((int64_t)kvh * nsp + sp) * G * kRecF;
    for (int hr = 0; hr < G; hr += kMergeH) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < HPL; i++) {
            const int h = (lane >> 4) + 4 * i;
            if (h < G && h >= hr && h < hr + kMergeH) {
                if ((lane & 15) == 0) { s_m[wave][h] = m_run[i]; s_l[wave][h] = lsum[i]; }
                float* dst = s_buf + (wave * kMergeH + h - hr) * kHd + 8 * (lane & 15);
                *reinterpret_cast<f4_t*>(dst) = f4_t{o[0][i], o[1][i], o[2][i], o[3][i]};
                *reinterpret_cast<f4_t*>(dst + 4) = f4_t{o[4][i], o[5][i], o[6][i], o[7][i]};
            }
        }
        __syncthreads();
        const int nh = G - hr < kMergeH ? G - hr : kMergeH;
        for (int idx = tid; idx < nh * kHd; idx += kAW * 64) {
            const int h = hr + idx / kHd, d = idx % kHd;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < kAW; w++) M = fmaxf(M, s_m[w][h]);
            float L = 0.f, Ov = 0.f;
#pragma unroll
            for (int w = 0; w < kAW; w++) {
                const float f = s_m[w][h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[w][h] - M);
                L += s_l[w][h] * f;
                Ov += s_buf[(w * kMergeH + h - hr) * kHd + d] * f;
            }
            __hip_atomic_store(rec + h * kRecF + 4 + d, Ov, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d == 0) {
                __hip_atomic_store(rec + h * kRecF, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(rec + h * kRecF + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    // Publication.  The records are agent-scope atomic stores; each thread
    // waits for its own to complete (the barrier itself waits only for LDS
    // traffic), the workgroup barrier orders all of them before thread 0's
    // counter increment, and that increment is a release at agent scope (L2
    // written back, thread 0's stores complete).  The workgroup that takes the
    // last increment acquires at agent scope (its L2 copy invalidated) before
    // it reads the records: release / acquire through the counter.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t* ctr = A.counter + kvh * kCtrStride;
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == (uint32_t)(nsp - 1);
    }
    __syncthreads();
    if (!s_last) return;
    // ---- the last workgroup of this kv head merges every split.  One
    // device-scope acquire (this XCD's L2 drops its non-coherent lines) makes
    // the other workgroups' write-through records visible to plain loads,
    // which are issued unconditionally (clamped indices, zero weights past the
    // end) so that each thread's loads go out as one batch.
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const float* r0 = A.rec + (int64_t)kvh * nsp * G * kRecF;
    if (nsp <= 32) {
        // One wave per query head, no workgroup barrier: lane p (< nsp) holds
        // split p's (m, l); lane (half, dq) sums the O rows of splits half,
        // half + 2, ... over dimensions 4 dq .. 4 dq + 3.  Every load (split
        // maxima included) is issued before the first wait.
        const int half = lane >> 5, dq = lane & 31;
        for (int h = wave; h < G; h += kAW) {
            const int pl = lane < nsp ? lane : nsp - 1;
            const f4_t ml = *reinterpret_cast<const f4_t*>(r0 + (int64_t)(pl * G + h) * kRecF);
            f4_t ov[16];
            float mo[16];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int p = half + 2 * j;
                const int pc = p < nsp ? p : nsp - 1;
                ov[j] = *reinterpret_cast<const f4_t*>(r0 + (int64_t)(pc * G + h) * kRecF + 4 + 4 * dq);
                mo[j] = r0[(int64_t)(pc * G + h) * kRecF];
            }
            float M = lane < nsp ? ml[0] : -INFINITY;
#pragma unroll
            for (int o2 = 32; o2 > 0; o2 >>= 1) M = fmaxf(M, __shfl_xor(M, o2, 64));
            float L = (lane < nsp && ml[0] != -INFINITY) ? __builtin_amdgcn_exp2f(ml[0] - M) * ml[1] : 0.f;
#pragma unroll
            for (int o2 = 32; o2 > 0; o2 >>= 1) L += __shfl_xor(L, o2, 64);
            f4_t acc = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int p = half + 2 * j;
                const float f = (p < nsp && mo[j] != -INFINITY) ? __builtin_amdgcn_exp2f(mo[j] - M) : 0.f;
                acc += ov[j] * f;
            }
#pragma unroll
            for (int c = 0; c < 4; c++) acc[c] += __shfl_xor(acc[c], 32, 64);
            if (half == 0) {
                const float inv = 1.f / L;
                uint16_t* op = A.out + (kvh * G + h) * kHd + 4 * dq;
                *reinterpret_cast<uint2*>(op) =
                    make_uint2((uint32_t)f2h(acc[0] * inv) | ((uint32_t)f2h(acc[1] * inv) << 16),
                               (uint32_t)f2h(acc[2] * inv) | ((uint32_t)f2h(acc[3] * inv) << 16));
            }
        }
        if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    float* s_cm = s_buf;
    float* s_cf = s_cm + kMaxRec;
    float* s_cl = s_cf + kMaxRec;
    f4_t* s_part = reinterpret_cast<f4_t*>(s_cl + kMaxRec);
    const int ne = nsp * G;
    constexpr int kMU = 12;                      // o rows in flight per thread
    const int ng = G * (kHd / 4);                // float4 groups of the outputs
    const int tpg = ng >= kAW * 64 ? 1 : kAW * 64 / ng;   // threads per group, each a stride of the splits
    // When every thread's O rows fit one batch (the usual case), they are
    // loaded together with the (m, l) words, before any wait: one memory
    // round trip instead of two.
    const bool one_batch = ng * tpg <= kAW * 64 && nsp <= kMU * tpg;   // uniform
    f4_t v0[kMU];
    {
        const int it = tid < ng * tpg ? tid : 0;
        const int gi = it % ng, sub = it / ng;
        const int h = gi / (kHd / 4), d4 = gi % (kHd / 4);
        if (one_batch) {
#pragma unroll
            for (int k = 0; k < kMU; k++) {
                const int p = sub + k * tpg;
                const int pc = p < nsp ? p : nsp - 1;
                v0[k] = *reinterpret_cast<const f4_t*>(r0 + (int64_t)(pc * G + h) * kRecF + 4 + 4 * d4);
            }
        }
    }
    for (int i = tid; i < ne; i += kAW * 64) {
        const f4_t h4 = *reinterpret_cast<const f4_t*>(r0 + (int64_t)i * kRecF);
        s_cm[i] = h4[0];
        s_cl[i] = h4[1];
    }
    __syncthreads();
    for (int h = wave; h < G; h += kAW) {
        float M = -INFINITY;
        for (int p = lane; p < nsp; p += 64) M = fmaxf(M, s_cm[p * G + h]);
        for (int o2 = 32; o2 > 0; o2 >>= 1) M = fmaxf(M, __shfl_xor(M, o2, 64));
        float L = 0.f;
        for (int p = lane; p < nsp; p += 64) {
            const float mp = s_cm[p * G + h];
            const float f = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - M);
            s_cf[p * G + h] = f;
            L += f * s_cl[p * G + h];
        }
        for (int o2 = 32; o2 > 0; o2 >>= 1) L += __shfl_xor(L, o2, 64);
        if (lane == 0) s_L[h] = L;
    }
    __syncthreads();
    if (one_batch) {
        if (tid < ng * tpg) {
            const int gi = tid % ng, sub = tid / ng;
            const int h = gi / (kHd / 4);
            f4_t acc = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < kMU; k++) {
                const int p = sub + k * tpg;
                const float f = p < nsp ? s_cf[p * G + h] : 0.f;
                acc += v0[k] * f;
            }
            s_part[tid] = acc;
        }
    } else {
        for (int it = tid; it < ng * tpg; it += kAW * 64) {
            const int gi = it % ng, sub = it / ng;
            const int h = gi / (kHd / 4), d4 = gi % (kHd / 4);
            f4_t acc = f4_t{0.f, 0.f, 0.f, 0.f};
            for (int p0 = sub; p0 < nsp; p0 += kMU * tpg) {
                f4_t v[kMU];
                float f[kMU];
#pragma unroll
                for (int k = 0; k < kMU; k++) {
                    const int p = p0 + k * tpg;
                    const int pc = p < nsp ? p : nsp - 1;
                    v[k] = *reinterpret_cast<const f4_t*>(r0 + (int64_t)(pc * G + h) * kRecF + 4 + 4 * d4);
                    f[k] = p < nsp ? s_cf[pc * G + h] : 0.f;
                }
#pragma unroll
                for (int k = 0; k < kMU; k++) acc += v[k] * f[k];
            }
            s_part[it] = acc;
        }
    }
    __syncthreads();
    for (int gi = tid; gi < ng; gi += kAW * 64) {
        f4_t acc = s_part[gi];
        for (int sub = 1; sub < tpg; sub++) acc += s_part[gi + sub * ng];
        const int h = gi / (kHd / 4), d4 = gi % (kHd / 4);
        const float inv = 1.f / s_L[h];
        uint16_t* op = A.out + (kvh * G + h) * kHd + 4 * d4;
        const uint2 w = make_uint2((uint32_t)f2h(acc[0] * inv) | ((uint32_t)f2h(acc[1] * inv) << 16),
                                   (uint32_t)f2h(acc[2] * inv) | ((uint32_t)f2h(acc[3] * inv) << 16));
        *reinterpret_cast<uint2*>(op) = w;
    }
    __syncthreads();
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Splits (workgroups) per kv head: enough for the prefix at kWaveTiles tiles
// per wave, more when that leaves the 256 CUs idle (down to one tile per
// wave); the tail's tiles ride along (a wave may take a few more).
int64_t n_splits(int64_t n_heads, int group, int64_t t_prefix, int64_t t_tail) {
    const int64_t np = (t_prefix + kTile - 1) / kTile, nt = (t_tail + kTile - 1) / kTile;
    const int64_t tiles = np > 0 ? np : nt;
    int64_t n = (tiles + (int64_t)kAW * kWaveTiles - 1) / ((int64_t)kAW * kWaveTiles);
    int64_t fill = (256 + n_heads - 1) / n_heads;
    const int64_t most = (tiles + kAW - 1) / kAW;
    if (fill > kMaxRec / group) fill = kMaxRec / group;   // the merge stages nsp * group records
    if (n < fill) n = fill < most ? fill : most;
    // the merge takes at most kMaxRec records: longer prefixes give each
    // split's waves more tiles (tiles are dealt dynamically) instead of more splits
    if (n > kMaxRec / group) n = kMaxRec / group;
    return n > 0 ? n : 1;
}

bool res_ok(const lq_resident* r) {
    return r && r->a && r->b && r->mask && r->meta && r->scale && r->n_exc && r->status && r->n_heads > 0 &&
           r->cap_blocks > 0 && r->exc_cap >= 0;
}

int attention_launch(const lq_resident* k, const lq_resident* v, int64_t t_prefix, const uint16_t* d_q, int group,
                     const uint16_t* d_tail_k, const uint16_t* d_tail_v, int64_t t_tail, uint32_t* counters,
                     float* records, uint16_t* d_out, hipStream_t s);

// Static scratch layout: a fixed region of completion counters for up to
// kScratchHeads kv heads (so records of one geometry never land on counters
// another geometry uses), then the split records.
constexpr int64_t kScratchHeads = 1024;
constexpr int64_t kScratchCounterBytes = kScratchHeads * kCtrStride * 4;

// Scratch of lq_resident_attention_noalloc: the completion counters and split
// records of one decode step, one copy per device, held until the process
// ends.  In host code `scratch` names a host-side stand-in, never the device
// memory: kernels get the address hipGetSymbolAddress returns for the device.
static __device__ __align__(256) uint8_t scratch[LQ_RES_ATTN_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];   // device address of `scratch` per device, null until set up

__global__ void k_zero_u32(uint32_t* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// Device address of the current device's scratch array.  On the first call
// per device: look it up and clear its counter region (a fill kernel on s,
// stream-ordered before the caller's launch; the counters must start at zero
// and every completed step leaves them zero; the split records are written
// before they are read).
int scratch_ptr(void** out, hipStream_t s) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return LQ_ERR_ARG;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return LQ_ERR_LAUNCH;
        hipLaunchKernelGGL(k_zero_u32, dim3(256), dim3(256), 0, s, static_cast<uint32_t*>(p),
                           kScratchCounterBytes / 4);
        if (hipGetLastError() != hipSuccess) return LQ_ERR_LAUNCH;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return LQ_OK;
}

}  // namespace

extern "C" {

int64_t lq_resident_workspace(int64_t n_heads, int64_t t_tokens) {
    if (n_heads <= 0 || t_tokens <= 0 || t_tokens % kRB) return -1;
    return n_heads * (t_tokens / kRB) * (int64_t)sizeof(uint32_t);
}

int lq_resident_quantize(const void* d_x, int dtype, int64_t n_heads, int64_t t_tokens, const float* d_scale32,
                         const uint16_t* d_scale16, const lq_resident* r, int64_t h0, int64_t blk0, void* d_work,
                         hipStream_t s) {
    if (!d_x || !d_scale32 || !d_scale16 || !res_ok(r) || !d_work || dtype < 0 || dtype > 2 || n_heads <= 0 ||
        t_tokens <= 0 || t_tokens % kRB || h0 < 0 || blk0 < 0)
        return LQ_ERR_ARG;
    const int64_t nb = t_tokens / kRB;
    if (h0 + n_heads > r->n_heads || blk0 + nb > r->cap_blocks || nb > INT_MAX || n_heads > 65535) return LQ_ERR_ARG;
    uint32_t* cnt = static_cast<uint32_t*>(d_work);
    const dim3 grid((unsigned)nb, (unsigned)n_heads);
    hipLaunchKernelGGL(k_res_quant, grid, dim3(256), 0, s, d_x, dtype, t_tokens, d_scale32, d_scale16, *r, h0, blk0,
                       cnt);
    hipLaunchKernelGGL(k_res_scan, dim3(1), dim3(256), 0, s, cnt, nb, n_heads, *r, h0, blk0);
    hipLaunchKernelGGL(k_res_fill, grid, dim3(256), 0, s, d_x, dtype, t_tokens, d_scale32, *r, h0, blk0);
    return launch_status();
}

int lq_resident_dequant(const lq_resident* r, int64_t h0, int64_t n_heads, int64_t blk0, int64_t n_blocks,
                        void* d_out, int out_dtype, hipStream_t s) {
    if (!res_ok(r) || !d_out || out_dtype < 0 || out_dtype > 2 || h0 < 0 || n_heads <= 0 || blk0 < 0 ||
        n_blocks <= 0 || h0 + n_heads > r->n_heads || blk0 + n_blocks > r->cap_blocks || n_heads > 65535 ||
        n_blocks > INT_MAX)
        return LQ_ERR_ARG;
    hipLaunchKernelGGL(k_res_dequant, dim3((unsigned)n_blocks, (unsigned)n_heads), dim3(256), 0, s, *r, h0, blk0,
                       n_blocks, d_out, out_dtype);
    return launch_status();
}

int64_t lq_resident_attn_workspace(int64_t n_heads, int group, int64_t t_prefix, int64_t t_tail) {
    if (n_heads <= 0 || group < 1 || group > 16 || t_prefix < 0 || t_tail < 0 || t_prefix + t_tail <= 0) return -1;
    const int64_t nsp = n_splits(n_heads, group, t_prefix, t_tail);
    if (nsp * group > kMaxRec) return -1;
    const int64_t counters = n_heads * kCtrStride * 4;
    return counters + n_heads * nsp * group * kRecF * (int64_t)sizeof(float);
}

int lq_resident_attention(const lq_resident* k, const lq_resident* v, int64_t t_prefix, const uint16_t* d_q,
                          int group, const uint16_t* d_tail_k, const uint16_t* d_tail_v, int64_t t_tail,
                          void* d_work, uint16_t* d_out, hipStream_t s) {
    if (!d_work || !k || k->n_heads <= 0) return LQ_ERR_ARG;
    uint32_t* counters = static_cast<uint32_t*>(d_work);
    float* records = reinterpret_cast<float*>(static_cast<char*>(d_work) + k->n_heads * kCtrStride * 4);
    return attention_launch(k, v, t_prefix, d_q, group, d_tail_k, d_tail_v, t_tail, counters, records, d_out, s);
}

int lq_resident_attention_noalloc(const lq_resident* k, const lq_resident* v, int64_t t_prefix, const uint16_t* d_q,
                                  int group, const uint16_t* d_tail_k, const uint16_t* d_tail_v, int64_t t_tail,
                                  uint16_t* d_out, hipStream_t s) {
    // size check first, from the host-side geometry alone: an oversize step is
    // refused before any HIP call
    if (!k || k->n_heads <= 0) return LQ_ERR_ARG;
    const int64_t need = lq_resident_attn_workspace(k->n_heads, group, t_prefix, t_tail);
    if (need < 0) return LQ_ERR_ARG;
    const int64_t rec_bytes = need - k->n_heads * kCtrStride * 4;
    if (k->n_heads > kScratchHeads || rec_bytes > (int64_t)LQ_RES_ATTN_SCRATCH_BYTES - kScratchCounterBytes)
        return LQ_ERR_SCRATCH;
    void* p = nullptr;
    const int rc = scratch_ptr(&p, s);
    if (rc != LQ_OK) return rc;
    return attention_launch(k, v, t_prefix, d_q, group, d_tail_k, d_tail_v, t_tail, static_cast<uint32_t*>(p),
                            reinterpret_cast<float*>(static_cast<char*>(p) + kScratchCounterBytes), d_out, s);
}

}  // extern "C"

namespace {

// Argument checks and launch of k_res_attn with its completion counters (one
// per kv head, kCtrStride apart, zero on entry and left zero) and split records.
int attention_launch(const lq_resident* k, const lq_resident* v, int64_t t_prefix, const uint16_t* d_q, int group,
                     const uint16_t* d_tail_k, const uint16_t* d_tail_v, int64_t t_tail, uint32_t* counters,
                     float* records, uint16_t* d_out, hipStream_t s) {
    if (!d_q || !d_out || !counters || !records || group < 1 || group > 16 || t_prefix < 0 || t_tail < 0 ||
        t_prefix + t_tail <= 0 || t_prefix % kRB)
        return LQ_ERR_ARG;
    if (t_tail > 0 && (!d_tail_k || !d_tail_v)) return LQ_ERR_ARG;
    if (t_prefix > 0 && (!res_ok(k) || !res_ok(v) || k->n_heads != v->n_heads || k->cap_blocks != v->cap_blocks ||
                         t_prefix / kRB > k->cap_blocks ||
                         t_prefix / kRB > v->cap_blocks))
        return LQ_ERR_ARG;
    int64_t n_heads = t_prefix > 0 ? k->n_heads : -1;
    if (n_heads <= 0) {
        if (!k || k->n_heads <= 0) return LQ_ERR_ARG;
        n_heads = k->n_heads;
    }
    AttnArgs A{};
    if (t_prefix > 0) { A.k = *k; A.v = *v; }
    A.t_prefix = t_prefix;
    A.t_tail = t_tail;
    A.q = d_q;
    A.tail_k = d_tail_k;
    A.tail_v = d_tail_v;
    A.group = group;
    A.nsp = (int)n_splits(n_heads, group, t_prefix, t_tail);
    A.counter = counters;
    A.rec = records;
    A.out = d_out;
    const int64_t grid = n_heads * A.nsp;
    if (grid > INT_MAX || (int64_t)A.nsp * group > kMaxRec) return LQ_ERR_ARG;
    const int hpl = (group + 3) / 4;
    switch (hpl) {
        case 1: hipLaunchKernelGGL(k_res_attn<1>, dim3((unsigned)grid), dim3(kAW * 64), 0, s, A); break;
        case 2: hipLaunchKernelGGL(k_res_attn<2>, dim3((unsigned)grid), dim3(kAW * 64), 0, s, A); break;
        case 3: hipLaunchKernelGGL(k_res_attn<3>, dim3((unsigned)grid), dim3(kAW * 64), 0, s, A); break;
        default: hipLaunchKernelGGL(k_res_attn<4>, dim3((unsigned)grid), dim3(kAW * 64), 0, s, A); break;
    }
    return launch_status();
}

}  // namespace

extern "C" {

}  // extern "C"
