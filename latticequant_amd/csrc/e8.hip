// E8 lattice kernels for gfx950: nearest-point search, symbolisation,
// per-head scales and the chunk quantizer of the compressed-KV write path.
#include <climits>

#include "lq_scales.h"

using namespace lq;

namespace {

// ------------------------------------------------------------ encode API --

__global__ void k_e8_encode(const float* __restrict__ x, int64_t n, int mode, float* __restrict__ out) {
    int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n) return;
    float xv[8], r[8];
    load8(x, LQ_F32, v, xv);
    if (mode == 1) {
        d8_round(xv, r);
    } else {
        int cos = e8_nearest_fast(xv, r);
        float off = cos ? 0.5f : 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) r[i] = r[i] + off;
    }
    store8(out, LQ_F32, v, r);
}

// e8_to_symbols (core/entropy_coder.py:46-68) on arbitrary float points.
__global__ void k_e8_to_symbols(const float* __restrict__ q, int64_t n, int32_t* __restrict__ coset,
                                int32_t* __restrict__ sym8) {
    int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n) return;
    float p[8];
    load8(q, LQ_F32, v, p);
    int half = fabsf(p[0] - rintf(p[0])) > 0.25f;
    coset[v] = half;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float t = half ? p[i] - 0.5f : p[i];
        int32_t c = (int32_t)rintf(t);
        sym8[8 * v + i] = i < 7 ? c : (c >> 1);   // floor(c7 / 2)
    }
}

// symbols_to_e8 (core/entropy_coder.py:71-89).
__global__ void k_symbols_to_e8(const int32_t* __restrict__ coset, const int32_t* __restrict__ sym8, int64_t n,
                                float* __restrict__ q) {
    int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n) return;
    const int32_t* s = sym8 + 8 * v;
    int32_t sum7 = 0;
    float o[8];
    float off = coset[v] == 1 ? 0.5f : 0.f;
#pragma unroll
    for (int i = 0; i < 7; i++) { sum7 += s[i]; o[i] = (float)s[i] + off; }
    o[7] = (float)(2 * s[7] + (sum7 & 1)) + off;
    store8(q, LQ_F32, v, o);
}

// x / scale[head] -> nearest E8 point (fp32), head = v / bph; the
// quantizer of _compress_tensor (llm/compressed_kv_cache.py:199-201) without
// symbolisation, for the fixed-rate path.
__global__ void k_quantize_heads(const void* __restrict__ x, int dtype, int64_t n, int64_t bph,
                                 const float* __restrict__ scale32, const int32_t* __restrict__ fastdiv,
                                 float* __restrict__ q) {
    int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n) return;
    const int64_t h = v / bph;
    const float s = scale32[h];
    const int32_t fw = fastdiv[h];
    const bool fast = fw != 0;
    const float rs = __int_as_float(fw);   // RN(1 / s) when fast
    float xv[8], t[8], ic[8];
    load8(x, dtype, v, xv);
#pragma unroll
    for (int i = 0; i < 8; i++) t[i] = div_scaled(xv[i], s, rs, fast);
    const float off = e8_nearest_fast(t, ic) ? 0.5f : 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) ic[i] = ic[i] + off;
    store8(q, LQ_F32, v, ic);
}

// ---------------------------------------------------------- head scales --

// Partial sums of x^2 per head in double: grid (heads, parts).  ROT: of the
// forward-rotated rows (lq_scales.h head_sumsq_part); LPR > 0: lpr known.
template <bool ROT, int LPR = 0>
__global__ void k_head_sumsq(const void* __restrict__ x, int dtype, int64_t vec_per_head, int parts,
                             double* __restrict__ work, const float* __restrict__ signs, int lpr, float rdiv) {
    __shared__ double red[256];
    head_sumsq_part<ROT, LPR>(x, dtype, vec_per_head, parts, blockIdx.x, blockIdx.y, work, red, signs, lpr, rdiv);
}

__device__ void fastdiv_check(float s, int32_t* word) {
    __shared__ int bad;
    const int32_t w = fastdiv_word(s, &bad);
    if (threadIdx.x == 0) *word = w;
}

// sigma^2, scales (llm/compressed_kv_cache.py:189-196) and fast-division flag.
__global__ void k_head_finalize(const double* __restrict__ work, int parts, int64_t elems_per_head,
                                int64_t n_heads, const int32_t* __restrict__ chunk_bits, int dtype,
                                float* __restrict__ sigma2, float* __restrict__ scale32,
                                uint16_t* __restrict__ scale16, int32_t* __restrict__ fastdiv) {
    int64_t h = blockIdx.x;
    __shared__ float sc;
    if (threadIdx.x == 0) {
        double acc = 0.0;
        for (int p = 0; p < parts; p++) acc += work[h * parts + p];
        float s2;
        const float s = head_scale(acc, elems_per_head, chunk_bits[h / n_heads], &s2);
        sigma2[h] = s2;
        scale32[h] = s;
        scale16[h] = f2h(s);
        sc = s;
    }
    __syncthreads();
    if (dtype == LQ_F16) {
        fastdiv_check(sc, fastdiv + h);
    } else if (threadIdx.x == 0) {
        fastdiv[h] = 0;
    }
}

__global__ void k_scale_fastdiv(const float* __restrict__ scale32, int dtype, int32_t* __restrict__ fastdiv) {
    int64_t h = blockIdx.x;
    if (dtype == LQ_F16) {
        fastdiv_check(scale32[h], fastdiv + h);
    } else if (threadIdx.x == 0) {
        fastdiv[h] = 0;
    }
}

// -------------------------------------------------------- chunk quantize --

constexpr int kQThreads = 256;
constexpr int kQBlocksPerWG = 8;
// LDS histogram row of one stream: 256 bins indexed by the symbol's low byte,
// padded so consecutive rows start 8 banks apart
constexpr int kHRow = 256 + 8;
constexpr int64_t kMaxBph = 1 << 30;   // vectors per head (2^27 tokens of 128 dims): in-head offsets stay int32

// One workgroup quantizes kQBlocksPerWG consecutive LQ_BLK-vector blocks of one
// chunk.  Per block it writes the coset bitmap (wave ballots, i.e. the
// reference's LSB-first pack_coset_bits layout), the coset-1 count and the
// symbols in the interleaved column layout of sym_pos (element index; int8
// symbols, or int16 for the wide path), staged in LDS so the global stores are
// 16-byte and contiguous.  int8: the 16 x 256 symbol histograms accumulate in
// LDS and are flushed once per workgroup; a symbol outside int8 sets
// LQ_ST_SYM_OVERFLOW (the chunk then needs the wide path).  int16: per-stream
// min / max instead (the histogram of the wide path is a second pass over the
// symbols, in the window the min fixes).
// DITHER: the chunk's dither (dither8, seed dseed[chunk]) is added to x / scale
// before the nearest-point search and taken off again in the dequantised output.
// Histogram of one staged 16-byte row: int8 symbols of vectors 16g .. 16g + 15
// of one coset's group g at one coordinate (the sym_pos layout).  Counting
// from the staged rows rather than per vector puts the lanes of one LDS atomic
// on 8 coordinates x 8 groups instead of one coordinate, so far fewer lanes
// meet on one bin (same-address atomics serialise).
__device__ __forceinline__ void stage_hist(const uint4& w, int row16, int n0, int n1, uint32_t* shist) {
    const int p = row16 * 16;
    const int r1 = sym_region(1, n0);
    const int c = p >= r1;
    const int q = p - (c ? r1 : 0);
    const int left = (c ? n1 : n0) - 16 * (q >> 7);   // vectors of this group, >= 1
    uint32_t* row = shist + (c * 8 + ((q >> 4) & 7)) * kHRow;
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    if (left >= 16) {
#pragma unroll
        for (int k = 0; k < 16; k++) atomicAdd(row + ((d[k >> 2] >> (8 * (k & 3))) & 255u), 1u);
    } else {
#pragma unroll
        for (int k = 0; k < 16; k++)
            if (k < left) atomicAdd(row + ((d[k >> 2] >> (8 * (k & 3))) & 255u), 1u);
    }
}

// Wide path: min / max of the int16 symbols of one staged 16-byte row (8
// symbols of one column), folded into the copying thread's running values of
// the row's coset.  Row j of the staging holds column (j / 2) % 8 of its coset
// region (regions start at multiples of 128 symbols, a column chunk spans two
// rows), so the rows a thread copies (j = tid + 256 k) share one coordinate.
// Rows past the column's count hold stale staging and are skipped.
typedef short short2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void stage_minmax(const uint4& w, int row16, int n0, int n1, int tmin[2], int tmax[2]) {
    const int e = row16 * 8;   // first symbol of the row
    const int r1 = sym_region(1, n0);
    const int c = e >= r1;
    const int q = e - (c ? r1 : 0);
    const int left = (c ? n1 : n0) - (16 * (q >> 7) + (q & 15));   // symbols of this column from the row on
    if (left <= 0) return;
    int lo, hi;
    if (left >= 8) {
        const short2_t a = __builtin_bit_cast(short2_t, w.x), b = __builtin_bit_cast(short2_t, w.y);
        const short2_t cc = __builtin_bit_cast(short2_t, w.z), d = __builtin_bit_cast(short2_t, w.w);
        const short2_t mn = __builtin_elementwise_min(__builtin_elementwise_min(a, b), __builtin_elementwise_min(cc, d));
        const short2_t mx = __builtin_elementwise_max(__builtin_elementwise_max(a, b), __builtin_elementwise_max(cc, d));
        lo = min((int)mn.x, (int)mn.y);
        hi = max((int)mx.x, (int)mx.y);
    } else {
        const uint32_t d[4] = {w.x, w.y, w.z, w.w};
        lo = INT_MAX;
        hi = INT_MIN;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int v = (int)(int16_t)(d[k >> 1] >> ((k & 1) * 16));
            if (k < left) { lo = min(lo, v); hi = max(hi, v); }
        }
    }
    if (c) { tmin[1] = min(tmin[1], lo); tmax[1] = max(tmax[1], hi); }
    else { tmin[0] = min(tmin[0], lo); tmax[0] = max(tmax[0], hi); }
}

// k_chunk_quantize (described above).  LEAN: the host guarantees bph >= LQ_BLK
// (a block spans at most two heads) and no dequantised output; the general
// paths are compiled out, which frees the scalar registers they held (fewer
// spills through VGPR lanes in the block loop).  ROT: the input rows are first
// rotated in registers (rht_lanes, sign row = the head, lpr lanes per row),
// exactly the fp32 values a materialised forward rotation holds, and divided
// by the scale as IEEE division rounds (div_exact where the row and the scale
// lie in its range); no dequantised output, at least 5 waves per SIMD.
// LDT >= 0: the input dtype as a compile-time constant (the lean launches),
// so no dtype test is kept live across the block loop.  LPR > 0: the rotation's
// lanes per row as a compile-time constant, so the butterfly stages are
// straight-line code (no per-stage branch and register copies).
template <typename SymT, bool DITHER, bool LEAN = false, bool ROT = false, int LDT = -1, int LPR = 0>
__global__ __launch_bounds__(kQThreads, ROT ? 5 : (LEAN ? 7 : 1)) void k_chunk_quantize(
    const void* __restrict__ x, int dtype, int64_t n_heads, int64_t bph, int64_t nblk,
    const float* __restrict__ scale32, const int32_t* __restrict__ fastdiv, SymT* __restrict__ sym,
    uint8_t* __restrict__ coset_bits, uint32_t* __restrict__ blk_n1, uint32_t* __restrict__ hist,
    int32_t* __restrict__ minmax, int32_t* __restrict__ status, void* __restrict__ deq, int deq_dtype,
    const int64_t* __restrict__ dseed, const float* __restrict__ signs, int lpr, float rdiv) {
    constexpr bool kWide = sizeof(SymT) == 2;
    constexpr int kSymMin = kWide ? -32768 : -128, kSymMax = kWide ? 32767 : 127;
    __shared__ uint32_t shist[kWide ? 1 : LQ_STREAMS * kHRow];
    __shared__ int smin[LQ_STREAMS], smax[LQ_STREAMS];
    __shared__ __align__(16) SymT stage[kSymStride];
    __shared__ __align__(16) unsigned long long masks[kBlk / 64];
    __shared__ int sflag;
    __shared__ __align__(16) float tslot[ROT ? 8 * kQThreads : 4];   // ROT: each lane's t for the exact path
    const float rrcp = ROT ? 1.0f / rdiv : 1.0f;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t wg_per_chunk = (nblk + kQBlocksPerWG - 1) / kQBlocksPerWG;
    const int64_t chunk = blockIdx.x / wg_per_chunk;
    const int64_t b0 = (blockIdx.x % wg_per_chunk) * kQBlocksPerWG;
    const int64_t V = n_heads * bph;

    if constexpr (!kWide) {
        for (int i = tid; i < LQ_STREAMS * kHRow; i += kQThreads) shist[i] = 0;
    }
    if (tid < LQ_STREAMS) { smin[tid] = INT_MAX; smax[tid] = INT_MIN; }
    if (tid == 0) sflag = 0;
    __syncthreads();
    // wide path: this thread's running min / max per coset of its coordinate
    // (stage_minmax: the staged rows a thread copies all hold one coordinate)
    int tmin[2] = {INT_MAX, INT_MAX}, tmax[2] = {INT_MIN, INT_MIN};

    int flag = 0;
    for (int bi = 0; bi < kQBlocksPerWG; bi++) {
        const int64_t blk = b0 + bi;
        if (blk >= nblk) break;
        const int64_t vbase = blk * kBlk;
        const int valid = (int)((V - vbase) < kBlk ? (V - vbase) : kBlk);
        // head of the block's first vector and its offset in that head (uniform);
        // a lane steps over the head boundaries its vector lies past
        const int64_t hblk = vbase / bph;
        const int rblk = (int)(vbase - hblk * bph);
        // with bph >= kBlk a block spans at most two heads: their scale,
        // reciprocal and fast-division flag are read once per block
        const bool two_heads = LEAN || bph >= kBlk;
        const int64_t hq0 = chunk * n_heads + hblk;
        const int64_t hq1 = hblk + 1 < n_heads ? hq0 + 1 : hq0;
        float s0 = 1.f, s1 = 1.f, rs0 = 1.f, rs1 = 1.f;
        bool f0 = false, f1 = false;
        if (two_heads) {
            s0 = scale32[hq0]; s1 = scale32[hq1];
            if (ROT) {    // rotated values are fp32: div_exact where in range
                rs0 = 1.0f / s0; rs1 = 1.0f / s1;
                f0 = s0 >= 0x1p-60f && s0 <= 0x1p60f;
                f1 = s1 >= 0x1p-60f && s1 <= 0x1p60f;
            } else {
                const int32_t w0 = fastdiv[hq0], w1 = fastdiv[hq1];
                f0 = w0 != 0; f1 = w1 != 0;
                rs0 = __int_as_float(w0); rs1 = __int_as_float(w1);   // RN(1 / s) where fast
            }
        }
        int32_t sy[2][8];
        int cs[2];
        unsigned long long bal[2];
        // pass 1: quantize two vectors per thread
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int vl = r * kQThreads + tid;
            cs[r] = 0;
            if (vl < valid) {
                const int64_t v = vbase + vl;
                float s, rs;
                bool fast;
                int64_t hq;
                if (two_heads) {
                    const bool nxt = rblk + vl >= (int)bph;
                    s = nxt ? s1 : s0;
                    rs = nxt ? rs1 : rs0;
                    fast = nxt ? f1 : f0;
                    hq = nxt ? hq1 : hq0;
                } else {
                    int rr = rblk + vl;
                    int64_t h = hq0;
                    while (rr >= (int)bph) { rr -= (int)bph; h++; }
                    s = scale32[h];
                    if (ROT) {
                        rs = 1.0f / s;
                        fast = s >= 0x1p-60f && s <= 0x1p60f;
                    } else {
                        const int32_t w = fastdiv[h];
                        rs = __int_as_float(w);
                        fast = w != 0;
                    }
                    hq = h;
                }
                float xv[8], t[8], ic[8], dd[8];
                load8(x, LDT >= 0 ? LDT : dtype, chunk * V + v, xv);
                if constexpr (ROT) {
                    // rows start at multiples of lpr vectors and blocks at
                    // multiples of 512, so the lane's place in its row is tid % lpr;
                    // valid is a multiple of lpr, so whole rows are live together
                    float sg[8];
                    const int lw = LPR > 0 ? LPR : lpr;
                    const int part = tid & (lw - 1);
                    load_signs8(signs + hq * (8 * (int64_t)lw) + 8 * part, sg);
                    // fp16 rows: no range test (every quotient is in range; the
                    // sign of a zero t does not change its lattice point)
                    const bool narrow = rht_lanes<LDT == LQ_F16>(xv, sg, part, lw, rdiv, rrcp, false);
                    if (fast && narrow) {
#pragma unroll
                        for (int i = 0; i < 8; i++) t[i] = div_exact(xv[i], s, rs);
                    } else {
#pragma unroll
                        for (int i = 0; i < 8; i++) t[i] = xv[i] / s;
                    }
                } else if (fast) {
#pragma unroll
                    for (int i = 0; i < 8; i++) t[i] = div_scaled(xv[i], s, rs, true);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) t[i] = div_scaled(xv[i], s, rs, false);
                }
                if constexpr (DITHER) {
                    dither8(mix64((uint64_t)dseed[chunk]), v, dd);
#pragma unroll
                    for (int i = 0; i < 8; i++) t[i] = t[i] + dd[i];
                }
                int c;
                float tm;   // max(1, max |t_i|)
                if constexpr (ROT) {
                    // the rotation is cross-lane, so the rare exact path cannot
                    // recompute t in a divergent branch: t waits in the lane's
                    // LDS slot instead of in registers
                    float4* slot = reinterpret_cast<float4*>(tslot + 8 * tid);
                    slot[0] = make_float4(t[0], t[1], t[2], t[3]);
                    slot[1] = make_float4(t[4], t[5], t[6], t[7]);
                    c = e8_nearest_fast(t, ic, [&](float tt[8]) {
                        asm volatile("" ::: "memory");   // read the slot back: t is not kept live for this
                        const float4 a = slot[0], b = slot[1];
                        tt[0] = a.x; tt[1] = a.y; tt[2] = a.z; tt[3] = a.w;
                        tt[4] = b.x; tt[5] = b.y; tt[6] = b.z; tt[7] = b.w;
                    }, &tm);
                } else {               // the rare exact path recomputes t from x
                    c = e8_nearest_fast(t, ic, [&](float tt[8]) {
                        float xx[8];
                        load8(x, LDT >= 0 ? LDT : dtype, chunk * V + v, xx);
#pragma unroll
                        for (int i = 0; i < 8; i++) tt[i] = div_scaled(xx[i], s, rs, fast);
                        if constexpr (DITHER) {
                            float d2[8];
                            dither8(mix64((uint64_t)dseed[chunk]), v, d2);
#pragma unroll
                            for (int i = 0; i < 8; i++) tt[i] = tt[i] + d2[i];
                        }
                    }, &tm);
                }
                cs[r] = c;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int32_t iv = (int32_t)ic[i];
                    sy[r][i] = i < 7 ? iv : (iv >> 1);
                }
                // max |t_i| < kSymMax - 1 puts every coordinate in
                // [-kSymMax, kSymMax] (e8_nearest_fast), so the symbols are in
                // range; only vectors with a larger (or infinite) |t_i| are
                // checked.  Out-of-range symbols are flagged and clamped
                // (histogram indices stay in range).
                if (!(tm < (float)(kSymMax - 1))) {
                    int32_t lo = INT_MAX, hi = INT_MIN;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        lo = min(lo, sy[r][i]);
                        hi = max(hi, sy[r][i]);
                    }
                    if (lo < kSymMin || hi > kSymMax) {
                        flag = 1;
#pragma unroll
                        for (int i = 0; i < 8; i++) sy[r][i] = min(max(sy[r][i], kSymMin), kSymMax);
                    }
                }
                if (!LEAN && !ROT && deq) {
                    float off = c ? 0.5f : 0.f, y[8];
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        if constexpr (DITHER) y[i] = ((ic[i] + off) - dd[i]) * s;
                        else y[i] = (ic[i] + off) * s;
                    }
                    store8(deq, deq_dtype, chunk * V + v, y);
                }
            }
            bal[r] = __ballot(cs[r]);
            if (lane == 0) masks[r * 4 + wave] = bal[r];
        }
        __syncthreads();
        // coset-1 counts of the block's 8 ballot words: the words are the same
        // for every lane, so they are made wave-uniform and counted on the
        // scalar unit
        int pc[kBlk / 64];
        int n1 = 0;
#pragma unroll
        for (int k = 0; k < kBlk / 64; k++) {
            const unsigned long long mk = masks[k];
            const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)mk);
            const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(mk >> 32));
            pc[k] = __builtin_popcount(lo) + __builtin_popcount(hi);
            n1 += pc[k];
        }
        const int n0 = valid - n1;
        // coset-1 vectors of the ballot words before this wave's (wave-uniform):
        // word r * 4 + wave.  Byte-wise prefix sums by one multiply (counts are
        // at most 64, three of them fit a byte) read at byte `wave`: scalar
        // arithmetic on the wave index, no per-word condition kept live.
        const uint32_t p0 = (uint32_t)pc[0] | ((uint32_t)pc[1] << 8) | ((uint32_t)pc[2] << 16);
        const uint32_t p1 = (uint32_t)pc[4] | ((uint32_t)pc[5] << 8) | ((uint32_t)pc[6] << 16);
        const uint32_t wsh = 8u * (uint32_t)wave;
        const int bef[2] = {(int)(((p0 * 0x01010100u) >> wsh) & 0xffu),
                            pc[0] + pc[1] + pc[2] + pc[3] + (int)(((p1 * 0x01010100u) >> wsh) & 0xffu)};
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int vl = r * kQThreads + tid;
            if (vl < valid) {
                const int before = bef[r];
                const unsigned long long m = bal[r];
                const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                int rank1 = before + below;
                int rank0 = vl - rank1;
                const int c = cs[r];
                const int rk = c ? rank1 : rank0;
                SymT* sp = stage + sym_pos(c, 0, rk, n0);   // column i adds 16 * i
                if constexpr (!kWide) {
#pragma unroll
                    for (int i = 0; i < 8; i++) sp[16 * i] = (SymT)sy[r][i];
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) sp[16 * i] = (SymT)sy[r][i];
                }
            }
        }
        __syncthreads();
        // copy-out: symbols, coset bitmap, block count
        {
            const int64_t gblk = chunk * nblk + blk;
            const int nbytes = (sym_region(1, n0) + 128 * ((n1 + 15) >> 4)) * (int)sizeof(SymT);
            uint4* dst = reinterpret_cast<uint4*>(sym + gblk * (int64_t)kSymStride);
            const uint4* src = reinterpret_cast<const uint4*>(stage);
            for (int i = tid; i * 16 < nbytes; i += kQThreads) {
                const uint4 w = src[i];
                dst[i] = w;
                if constexpr (!kWide) stage_hist(w, i, n0, n1, shist);
                else stage_minmax(w, i, n0, n1, tmin, tmax);
            }
            // the block's 64 bytes of coset bits as four 16-byte rows (lane offsets
            // shared with the copy above)
            uint4* cb = reinterpret_cast<uint4*>(coset_bits + gblk * (kBlk / 8));
            if (tid < kBlk / 128) cb[tid] = reinterpret_cast<const uint4*>(masks)[tid];
            if (tid == 0) blk_n1[gblk] = (uint32_t)n1;
        }
        __syncthreads();
    }
    if (flag) atomicOr(&sflag, 1);
    if constexpr (kWide) {   // this thread's coordinate, both cosets
        const int idx = (tid >> 1) & 7;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            if (tmin[c] != INT_MAX) atomicMin(&smin[c * 8 + idx], tmin[c]);
            if (tmax[c] != INT_MIN) atomicMax(&smax[c * 8 + idx], tmax[c]);
        }
    }
    __syncthreads();
    if constexpr (!kWide) {
        uint32_t* gh = hist + chunk * (LQ_STREAMS * 256);
        for (int i = tid; i < LQ_STREAMS * 256; i += kQThreads) {
            const uint32_t c = shist[(i >> 8) * kHRow + ((i & 255) ^ 128)];   // bin of symbol (i & 255) - 128
            if (c) atomicAdd(gh + i, c);
        }
    } else {
        if (tid < LQ_STREAMS && smax[tid] != INT_MIN) {
            atomicMin(minmax + (chunk * LQ_STREAMS + tid) * 2, smin[tid]);
            atomicMax(minmax + (chunk * LQ_STREAMS + tid) * 2 + 1, smax[tid]);
        }
    }
    if (tid == 0 && sflag) atomicOr(status + chunk, LQ_ST_SYM_OVERFLOW);
}

// Wide path, second pass: histograms of the int16 symbols in the window
// [min, min + 1023] of each stream (a stream whose max exceeds the window has
// an alphabet beyond L and is flagged by the table stage).  Workgroup: 16
// blocks x 16 streams of one chunk, one lane per (block, stream) column, read
// 16 symbols (32 bytes) at a time with the next chunk's loads in flight.
// Counts accumulate in LDS as 16-bit halves, two bins per word (a bin counts
// at most 16 x 512 symbols of a workgroup), and are added to hist once.
constexpr int kHBlocks = 16;

__global__ __launch_bounds__(256) void k_chunk_hist_wide(const int16_t* __restrict__ sym, const uint32_t* __restrict__ blk_n1,
                                                         int64_t nblk, int64_t V, const int32_t* __restrict__ minmax,
                                                         uint32_t* __restrict__ hist) {
    static_assert(kHBlocks * kBlk < 65536, "16-bit LDS counters");
    __shared__ uint32_t sh[LQ_STREAMS * LQ_L / 2];
    const int tid = threadIdx.x;
    const int64_t chunk = blockIdx.y;
    for (int i = tid; i < LQ_STREAMS * LQ_L / 2; i += 256) sh[i] = 0;
    __syncthreads();
    const int64_t g = (int64_t)blockIdx.x * kHBlocks + (tid >> 4);
    const int st = tid & 15;
    if (g < nblk) {
        const int c = st >> 3, idx = st & 7;
        const int64_t valid = V - g * kBlk < kBlk ? V - g * kBlk : kBlk;
        const int n1 = (int)blk_n1[chunk * nblk + g];
        const int n0 = (int)valid - n1;
        const int n = c ? n1 : n0;
        const int lo = minmax[(chunk * LQ_STREAMS + st) * 2];
        const int16_t* col = sym + (chunk * nblk + g) * (int64_t)kSymStride + sym_region(c, n0) + 16 * idx;
        uint32_t* hs = sh + st * (LQ_L / 2);
        const int nk = (n + 15) >> 4;   // column chunks (the last one may be partial)
        Chunk16<int16_t> cur = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)}, nxt = cur;
        if (nk > 0) cur = gload_chunk(col);
        for (int k = 0; k < nk; k++) {
            if (k + 1 < nk) nxt = gload_chunk(col + 128 * (int64_t)(k + 1));
            const int m = n - 16 * k < 16 ? n - 16 * k : 16;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int v = cur.get(i) - lo;
                if (i < m && (unsigned)v < (unsigned)LQ_L) atomicAdd(hs + (v >> 1), 1u << ((v & 1) * 16));
            }
            cur = nxt;
        }
    }
    __syncthreads();
    uint32_t* gh = hist + chunk * (LQ_STREAMS * LQ_L);
    for (int i = tid; i < LQ_STREAMS * LQ_L / 2; i += 256) {
        const uint32_t w = sh[i];
        if (w & 0xffffu) atomicAdd(gh + 2 * i, w & 0xffffu);
        if (w >> 16) atomicAdd(gh + 2 * i + 1, w >> 16);
    }
}

inline int launch_status() { return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_LAUNCH; }

}  // namespace

extern "C" {

int lq_e8_encode_f32(const float* d_x, int64_t n, int mode, float* d_out, hipStream_t s) {
    if (n < 0 || (mode != 0 && mode != 1)) return LQ_ERR_ARG;
    if (n == 0) return LQ_OK;
    hipLaunchKernelGGL(k_e8_encode, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_x, n, mode, d_out);
    return launch_status();
}

int lq_e8_to_symbols(const float* d_q, int64_t n, int32_t* d_coset, int32_t* d_sym8, hipStream_t s) {
    if (n < 0) return LQ_ERR_ARG;
    if (n == 0) return LQ_OK;
    hipLaunchKernelGGL(k_e8_to_symbols, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_q, n, d_coset, d_sym8);
    return launch_status();
}

int lq_symbols_to_e8(const int32_t* d_coset, const int32_t* d_sym8, int64_t n, float* d_q, hipStream_t s) {
    if (n < 0) return LQ_ERR_ARG;
    if (n == 0) return LQ_OK;
    hipLaunchKernelGGL(k_symbols_to_e8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_coset, d_sym8, n, d_q);
    return launch_status();
}

int lq_head_scales(const void* d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph,
                   const int32_t* d_chunk_bits, double* d_work, float* d_sigma2, float* d_scale32,
                   uint16_t* d_scale16, int32_t* d_fastdiv, hipStream_t s) {
    if (n_chunks <= 0 || n_heads <= 0 || bph <= 0 || dtype < 0 || dtype > 2) return LQ_ERR_ARG;
    const int64_t H = n_chunks * n_heads;
    const int parts = head_parts(H, bph);
    hipLaunchKernelGGL(k_head_sumsq<false>, dim3((unsigned)H, parts), dim3(256), 0, s, d_x, dtype, bph, parts, d_work,
                       nullptr, 1, 1.0f);
    hipLaunchKernelGGL(k_head_finalize, dim3((unsigned)H), dim3(256), 0, s, d_work, parts, bph * 8, n_heads,
                       d_chunk_bits, dtype, d_sigma2, d_scale32, d_scale16, d_fastdiv);
    return launch_status();
}

// Small updates without entropy coding: lq_head_scales, then the quantizer
// with the dequantised output; its symbol staging, bitmap, counts, histogram
// and status land in the caller's scratch and are not read (the histogram
// and status words need no clearing: they are only added to).
static inline int64_t qd_align(int64_t b) { return (b + 255) / 256 * 256; }

int64_t lq_quantize_deq_workspace(int64_t n_chunks, int64_t n_heads, int64_t bph) {
    if (n_chunks <= 0 || n_heads <= 0 || bph <= 0 || bph > kMaxBph) return -1;
    const int64_t H = n_chunks * n_heads, nblk = (n_heads * bph + kBlk - 1) / kBlk;
    return qd_align((4096 + H) * 8) + qd_align(H * 4) + qd_align(n_chunks * nblk * kSymStride) +
           qd_align(n_chunks * nblk * (kBlk / 8)) + qd_align(n_chunks * nblk * 4) +
           qd_align(n_chunks * LQ_STREAMS * 256 * 4) + qd_align(n_chunks * 4);
}

int lq_quantize_deq(const void* d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph,
                    const int32_t* d_chunk_bits, void* d_work, float* d_sigma2, float* d_scale32,
                    uint16_t* d_scale16, void* d_deq, hipStream_t s) {
    if (!d_x || !d_chunk_bits || !d_work || !d_sigma2 || !d_scale32 || !d_scale16 || !d_deq) return LQ_ERR_ARG;
    if (lq_quantize_deq_workspace(n_chunks, n_heads, bph) < 0 || dtype < 0 || dtype > 2) return LQ_ERR_ARG;
    const int64_t H = n_chunks * n_heads, nblk = (n_heads * bph + kBlk - 1) / kBlk;
    char* p = static_cast<char*>(d_work);
    double* work = reinterpret_cast<double*>(p);             p += qd_align((4096 + H) * 8);
    int32_t* fastdiv = reinterpret_cast<int32_t*>(p);        p += qd_align(H * 4);
    int8_t* sym = reinterpret_cast<int8_t*>(p);              p += qd_align(n_chunks * nblk * kSymStride);
    uint8_t* coset = reinterpret_cast<uint8_t*>(p);          p += qd_align(n_chunks * nblk * (kBlk / 8));
    uint32_t* n1 = reinterpret_cast<uint32_t*>(p);           p += qd_align(n_chunks * nblk * 4);
    uint32_t* hist = reinterpret_cast<uint32_t*>(p);         p += qd_align(n_chunks * LQ_STREAMS * 256 * 4);
    int32_t* status = reinterpret_cast<int32_t*>(p);
    const int rc = lq_head_scales(d_x, dtype, n_chunks, n_heads, bph, d_chunk_bits, work, d_sigma2, d_scale32,
                                  d_scale16, fastdiv, s);
    if (rc != LQ_OK) return rc;
    return lq_chunk_quantize(d_x, dtype, n_chunks, n_heads, bph, d_scale32, fastdiv, sym, coset, n1, hist, status,
                             d_deq, dtype, nullptr, s);
}

// Rotated rows (head_dim a power of two in [8, 128], bph a multiple of
// head_dim / 8): the scales of w = RHT(x) without materialising w; the
// fast-division flags are 0 (w is fp32).
int lq_head_scales_rht(const void* d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph, int head_dim,
                       const float* d_signs, const int32_t* d_chunk_bits, double* d_work, float* d_sigma2,
                       float* d_scale32, uint16_t* d_scale16, int32_t* d_fastdiv, hipStream_t s) {
    if (n_chunks <= 0 || n_heads <= 0 || bph <= 0 || dtype < 0 || dtype > 2 || !d_signs) return LQ_ERR_ARG;
    if (head_dim < 8 || head_dim > 128 || (head_dim & (head_dim - 1)) || bph % (head_dim / 8)) return LQ_ERR_ARG;
    const int64_t H = n_chunks * n_heads;
    const int parts = head_parts(H, bph);
    const float div = (float)sqrt((double)head_dim);
    if (head_dim == 128)
        hipLaunchKernelGGL((k_head_sumsq<true, 16>), dim3((unsigned)H, parts), dim3(256), 0, s, d_x, dtype, bph, parts,
                           d_work, d_signs, 16, div);
    else
        hipLaunchKernelGGL((k_head_sumsq<true, 0>), dim3((unsigned)H, parts), dim3(256), 0, s, d_x, dtype, bph, parts,
                           d_work, d_signs, head_dim / 8, div);
    hipLaunchKernelGGL(k_head_finalize, dim3((unsigned)H), dim3(256), 0, s, d_work, parts, bph * 8, n_heads,
                       d_chunk_bits, (int)LQ_F32, d_sigma2, d_scale32, d_scale16, d_fastdiv);
    return launch_status();
}

int lq_scale_fastdiv(const float* d_scale32, int64_t n_heads_total, int dtype, int32_t* d_fastdiv, hipStream_t s) {
    if (n_heads_total <= 0) return LQ_ERR_ARG;
    hipLaunchKernelGGL(k_scale_fastdiv, dim3((unsigned)n_heads_total), dim3(256), 0, s, d_scale32, dtype, d_fastdiv);
    return launch_status();
}

int lq_e8_quantize_heads(const void* d_x, int dtype, int64_t n_heads, int64_t bph, const float* d_scale32,
                         const int32_t* d_fastdiv, float* d_q, hipStream_t s) {
    if (n_heads <= 0 || bph <= 0 || dtype < 0 || dtype > 2) return LQ_ERR_ARG;
    const int64_t n = n_heads * bph;
    hipLaunchKernelGGL(k_quantize_heads, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_x, dtype, n, bph,
                       d_scale32, d_fastdiv, d_q);
    return launch_status();
}

int lq_chunk_quantize(const void* d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph,
                      const float* d_scale32, const int32_t* d_fastdiv, int8_t* d_sym, uint8_t* d_coset_bits,
                      uint32_t* d_blk_n1, uint32_t* d_hist, int32_t* d_status, void* d_deq, int deq_dtype,
                      const int64_t* d_dither_seed, hipStream_t s) {
    if (n_chunks <= 0 || n_heads <= 0 || bph <= 0 || bph > kMaxBph || dtype < 0 || dtype > 2) return LQ_ERR_ARG;
    const int64_t V = n_heads * bph;
    const int64_t nblk = (V + kBlk - 1) / kBlk;
    const int64_t wg = n_chunks * ((nblk + kQBlocksPerWG - 1) / kQBlocksPerWG);
    if (d_dither_seed)
        hipLaunchKernelGGL((k_chunk_quantize<int8_t, true>), dim3((unsigned)wg), dim3(kQThreads), 0, s, d_x, dtype,
                           n_heads, bph, nblk, d_scale32, d_fastdiv, d_sym, d_coset_bits, d_blk_n1, d_hist, nullptr,
                           d_status, d_deq, deq_dtype, d_dither_seed, nullptr, 1, 1.0f);
    else if (bph >= kBlk && !d_deq) {
#define LQ_LEAN(DT)                                                                                              \
        hipLaunchKernelGGL((k_chunk_quantize<int8_t, false, true, false, DT>), dim3((unsigned)wg), dim3(kQThreads),  \
                           0, s, d_x, dtype, n_heads, bph, nblk, d_scale32, d_fastdiv, d_sym, d_coset_bits, d_blk_n1, \
                           d_hist, nullptr, d_status, nullptr, deq_dtype, nullptr, nullptr, 1, 1.0f)
        if (dtype == LQ_F16) LQ_LEAN(LQ_F16);
        else if (dtype == LQ_BF16) LQ_LEAN(LQ_BF16);
        else LQ_LEAN(LQ_F32);
#undef LQ_LEAN
    }
    else
        hipLaunchKernelGGL((k_chunk_quantize<int8_t, false>), dim3((unsigned)wg), dim3(kQThreads), 0, s, d_x, dtype,
                           n_heads, bph, nblk, d_scale32, d_fastdiv, d_sym, d_coset_bits, d_blk_n1, d_hist, nullptr,
                           d_status, d_deq, deq_dtype, nullptr, nullptr, 1, 1.0f);
    return launch_status();
}

// Rotated rows: as lq_chunk_quantize on w = RHT(x) (sign row = the head,
// head_dim a power of two in [8, 128], bph a multiple of head_dim / 8), with
// the scale division rounded as IEEE division and no dequantised output.
int lq_chunk_quantize_rht(const void* d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph, int head_dim,
                          const float* d_signs, const float* d_scale32, int8_t* d_sym, uint8_t* d_coset_bits,
                          uint32_t* d_blk_n1, uint32_t* d_hist, int32_t* d_status, const int64_t* d_dither_seed,
                          hipStream_t s) {
    if (n_chunks <= 0 || n_heads <= 0 || bph <= 0 || bph > kMaxBph || dtype < 0 || dtype > 2 || !d_signs)
        return LQ_ERR_ARG;
    if (head_dim < 8 || head_dim > 128 || (head_dim & (head_dim - 1)) || bph % (head_dim / 8)) return LQ_ERR_ARG;
    const int64_t V = n_heads * bph;
    const int64_t nblk = (V + kBlk - 1) / kBlk;
    const int64_t wg = n_chunks * ((nblk + kQBlocksPerWG - 1) / kQBlocksPerWG);
    const float div = (float)sqrt((double)head_dim);
    const int lpr = head_dim / 8;
#define LQ_ROT(DI, LE, DT, LP)                                                                                    \
    hipLaunchKernelGGL((k_chunk_quantize<int8_t, DI, LE, true, DT, LP>), dim3((unsigned)wg), dim3(kQThreads), 0, s,  \
                       d_x, dtype, n_heads, bph, nblk, d_scale32, nullptr, d_sym, d_coset_bits, d_blk_n1, d_hist,      \
                       nullptr, d_status, nullptr, (int)LQ_F32, d_dither_seed, d_signs, lpr, div)
#define LQ_ROT_LP(DI, DT)                                                                                         \
    if (lpr == 16) LQ_ROT(DI, true, DT, 16);                                                                      \
    else LQ_ROT(DI, true, DT, 0)
#define LQ_ROT_DT(DI)                                                                                             \
    if (bph < kBlk) LQ_ROT(DI, false, -1, 0);                                                                     \
    else if (dtype == LQ_F16) { LQ_ROT_LP(DI, LQ_F16); }                                                          \
    else if (dtype == LQ_BF16) { LQ_ROT_LP(DI, LQ_BF16); }                                                        \
    else { LQ_ROT_LP(DI, LQ_F32); }
    if (d_dither_seed) { LQ_ROT_DT(true); }
    else { LQ_ROT_DT(false); }
#undef LQ_ROT_DT
#undef LQ_ROT_LP
#undef LQ_ROT
    return launch_status();
}

int lq_chunk_quantize_wide(const void* d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph,
                           const float* d_scale32, const int32_t* d_fastdiv, int16_t* d_sym, uint8_t* d_coset_bits,
                           uint32_t* d_blk_n1, int32_t* d_minmax, int32_t* d_status, void* d_deq, int deq_dtype,
                           const int64_t* d_dither_seed, hipStream_t s) {
    if (n_chunks <= 0 || n_heads <= 0 || bph <= 0 || bph > kMaxBph || dtype < 0 || dtype > 2 || !d_minmax)
        return LQ_ERR_ARG;
    const int64_t V = n_heads * bph;
    const int64_t nblk = (V + kBlk - 1) / kBlk;
    const int64_t wg = n_chunks * ((nblk + kQBlocksPerWG - 1) / kQBlocksPerWG);
    if (d_dither_seed)
        hipLaunchKernelGGL((k_chunk_quantize<int16_t, true>), dim3((unsigned)wg), dim3(kQThreads), 0, s, d_x, dtype,
                           n_heads, bph, nblk, d_scale32, d_fastdiv, d_sym, d_coset_bits, d_blk_n1, nullptr, d_minmax,
                           d_status, d_deq, deq_dtype, d_dither_seed, nullptr, 1, 1.0f);
    else if (bph >= kBlk && !d_deq) {
#define LQ_LEAN(DT)                                                                                               \
        hipLaunchKernelGGL((k_chunk_quantize<int16_t, false, true, false, DT>), dim3((unsigned)wg), dim3(kQThreads),  \
                           0, s, d_x, dtype, n_heads, bph, nblk, d_scale32, d_fastdiv, d_sym, d_coset_bits, d_blk_n1,  \
                           nullptr, d_minmax, d_status, nullptr, deq_dtype, nullptr, nullptr, 1, 1.0f)
        if (dtype == LQ_F16) LQ_LEAN(LQ_F16);
        else if (dtype == LQ_BF16) LQ_LEAN(LQ_BF16);
        else LQ_LEAN(LQ_F32);
#undef LQ_LEAN
    }
    else
        hipLaunchKernelGGL((k_chunk_quantize<int16_t, false>), dim3((unsigned)wg), dim3(kQThreads), 0, s, d_x, dtype,
                           n_heads, bph, nblk, d_scale32, d_fastdiv, d_sym, d_coset_bits, d_blk_n1, nullptr, d_minmax,
                           d_status, d_deq, deq_dtype, nullptr, nullptr, 1, 1.0f);
    return launch_status();
}

int lq_chunk_hist_wide(const int16_t* d_sym, const uint32_t* d_blk_n1, int64_t n_chunks, int64_t n_vectors,
                       const int32_t* d_minmax, uint32_t* d_hist, hipStream_t s) {
    if (n_chunks <= 0 || n_vectors <= 0 || !d_sym || !d_minmax || !d_hist) return LQ_ERR_ARG;
    const int64_t nblk = (n_vectors + kBlk - 1) / kBlk;
    hipLaunchKernelGGL(k_chunk_hist_wide, dim3((unsigned)((nblk + kHBlocks - 1) / kHBlocks), (unsigned)n_chunks),
                       dim3(256), 0, s, d_sym, d_blk_n1, nblk, n_vectors, d_minmax, d_hist);
    return launch_status();
}

}  // extern "C"
