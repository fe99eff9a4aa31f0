// Fixed-rate E8 storage kernels for gfx950 (b = 3, 4, 5 bits per dimension):
// pack / unpack + dequant and the single-pass repr / fallback merge.
//
// Layout (reference core/compact_storage.py:87-154): one big-endian b-byte
// word per vector, [coset(1) | c0..c6 (b each) | c7 >> 1 (b-1)], coordinates
// biased by R = 2^(b-1).  c7's low bit is recovered from the parity of
// c0 + .. + c6 (floor-mod, as unpack_e8 does).
#include "lq_scales.h"

using namespace lq;

namespace {

inline int launch_status() { return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_LAUNCH; }

__device__ __forceinline__ uint64_t load_be(const uint8_t* p, int bits) {
    uint64_t w = 0;
    for (int b = 0; b < bits; b++) w = (w << 8) | p[b];
    return w;
}

// decode one packed word into 8 fp32 lattice coordinates (coset offset applied)
__device__ __forceinline__ void unpack_word(uint64_t w, int bits, float q[8]) {
    const int R = 1 << (bits - 1);
    const uint64_t cm = (1ull << bits) - 1ull, um = (1ull << (bits - 1)) - 1ull;
    int c7u = (int)(w & um);
    w >>= (bits - 1);
    int c[7], ps = 0;
#pragma unroll
    for (int i = 6; i >= 0; i--) { c[i] = (int)(w & cm) - R; w >>= bits; }
    int coset = (int)(w & 1ull);
#pragma unroll
    for (int i = 0; i < 7; i++) ps += c[i];
    int c7 = c7u * 2 + (ps & 1) - R;
    float off = coset ? 0.5f : 0.f;
#pragma unroll
    for (int i = 0; i < 7; i++) q[i] = (float)c[i] + off;
    q[7] = (float)c7 + off;
}

__global__ void k_unpack(const uint8_t* __restrict__ packed, int bits, int64_t n, const float* __restrict__ scales,
                         int64_t n_scales, const int32_t* __restrict__ head_idx, uint16_t* __restrict__ out) {
    int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n) return;
    uint64_t w;
    if (bits == 4) {
        uint32_t u = reinterpret_cast<const uint32_t*>(packed)[v];
        w = __builtin_bswap32(u);
    } else {
        w = load_be(packed + v * bits, bits);
    }
    float q[8], y[8];
    unpack_word(w, bits, q);
    // an index outside [0, n_scales) is clamped: garbage out, never a fault
    const int64_t h = head_idx[v];
    float s = scales[h < 0 ? 0 : (h >= n_scales ? n_scales - 1 : h)];
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = q[i] * s;
    store8(out, LQ_F16, v, y);
}

// validate_e8 + pack_e8 for one point (core/compact_storage.py:39-154)
__global__ void k_pack(const float* __restrict__ q, int bits, int64_t n, uint8_t* __restrict__ packed,
                       int32_t* __restrict__ ok) {
    int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n) return;
    float p[8];
    load8(q, LQ_F32, v, p);
    float ri = 0.f, rh = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        ri = fmaxf(ri, fabsf(p[i] - rintf(p[i])));
        float h = p[i] - 0.5f;
        rh = fmaxf(rh, fabsf(h - rintf(h)));
    }
    const bool is_half = rh < 1e-5f, is_int = ri < 1e-5f;
    const int R = 1 << (bits - 1);
    int64_t sum = 0;
    bool good = is_half || is_int;
    uint64_t u[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int64_t c = (int64_t)rintf(is_half ? p[i] - 0.5f : p[i]);
        sum += c;
        good = good && c >= -R && c <= R - 1;
        u[i] = (uint64_t)(c + R);
    }
    good = good && ((sum & 1) == 0);
    uint64_t w = is_half ? 1ull : 0ull;
#pragma unroll
    for (int i = 0; i < 7; i++) w = (w << bits) | u[i];
    w = (w << (bits - 1)) | (u[7] >> 1);
    if (!good) w = 0;
    for (int b = bits - 1; b >= 0; b--) { packed[v * bits + b] = (uint8_t)(w & 0xff); w >>= 8; }
    ok[v] = good ? 1 : 0;
}

// ------------------------------------------------------------- merge ----
constexpr int kTile = 1024;
constexpr int kTileThreads = 1024;   // one vector per thread
constexpr int kTileRounds = kTile / kTileThreads;

// ------------------------------------------------ chained tile prefix --
//
// Decoupled look-back over kTile-vector tiles in start order: a workgroup
// takes a ticket (its tile), publishes the tile's count, then adds the counts
// of the tiles before it (64 at a time) until it meets one whose inclusive
// prefix is known.
// Tickets are taken in the order workgroups start, so every tile waited on is
// running or done and none of them waits on a later tile: the chain drains.
// status[] and the ticket counter must be zero before the launch (k_zero64);
// a wait that exceeds kSpinLimit polls sets *err instead of hanging.
constexpr uint64_t kStAgg = 1ull << 62, kStIncl = 2ull << 62, kStVal = (1ull << 62) - 1ull;
constexpr uint32_t kSpinLimit = 1u << 22;

__device__ __forceinline__ void st_status(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave 0 (all 64 lanes) only: exclusive prefix of tile t's count.  The lanes
// read the 64 status words before the current window end at once; the window
// is summed up to the nearest tile whose inclusive prefix is known, and moved
// back by 64 tiles when it holds only aggregates.
__device__ int64_t tile_lookback(uint64_t* status, int64_t t, int64_t count, int32_t* err) {
    const int lane = threadIdx.x & 63;
    if (t == 0) {
        if (lane == 0) st_status(status, kStIncl | (uint64_t)count);
        return 0;
    }
    if (lane == 0) st_status(status + t, kStAgg | (uint64_t)count);
    int64_t excl = 0, end = t;   // window: tiles end - 64 .. end - 1, lane j reads end - 1 - j
    uint32_t spins = 0;
    while (end > 0) {
        const int64_t j = end - 1 - lane;
        const uint64_t st = j >= 0 ? __hip_atomic_load(status + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : kStIncl;
        const uint64_t incl = __ballot((st >> 62) == 2);
        const int first = incl ? __builtin_ctzll(incl) : 64;   // nearest inclusive prefix in the window
        const uint64_t notready = __ballot((st >> 62) == 0) & (first < 64 ? (2ull << first) - 1ull : ~0ull);
        if (notready) {   // a tile before the nearest inclusive one has not published yet
            if (++spins > kSpinLimit) {
                if (lane == 0) atomicOr(err, 1);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            continue;
        }
        int64_t v = lane <= first && j >= 0 ? (int64_t)(st & kStVal) : 0;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        excl += v;
        if (first < 64) break;
        end -= 64;
    }
    if (lane == 0) st_status(status + t, kStIncl | (uint64_t)(excl + count));
    return excl;
}

// Clears p[0 .. n) and, when given, the one word *extra (an error word kept
// beside the caller's totals).
__global__ void k_zero64(uint64_t* __restrict__ p, int64_t n, int64_t* __restrict__ extra) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0ull;
    if (extra && blockIdx.x == 0 && threadIdx.x == 0) *extra = 0;
}

// sigma^2 partial sums per (head, part), exactly as lq_head_scales forms them
// (lq_scales.h head_sumsq_part, same part count), and, on the side, the clear
// of the fixed-rate encoder's look-back words clear[0 .. n_clear) and *extra.
__global__ __launch_bounds__(256) void k_compact_sumsq(const void* __restrict__ x, int dtype, int64_t bph, int parts,
                                                       double* __restrict__ work, uint64_t* __restrict__ clear,
                                                       int64_t n_clear, int64_t* __restrict__ extra) {
    __shared__ double red[256];
    const int64_t wg = (int64_t)blockIdx.y * gridDim.x + blockIdx.x, n_wg = (int64_t)gridDim.x * gridDim.y;
    for (int64_t i = wg * 256 + threadIdx.x; i < n_clear; i += n_wg * 256) clear[i] = 0ull;
    if (wg == 0 && threadIdx.x == 0) *extra = 0;
    head_sumsq_part<false>(x, dtype, bph, parts, blockIdx.x, blockIdx.y, work, red, nullptr, 1, 1.0f);
}

// One tile of kTile blocks per workgroup; ranks from the tile offset plus
// wave ballots, then either unpack the packed word or copy the fp16 fallback.
// LB: the tile offsets come from the chained look-back (tile = ticket order)
// instead of tile_off (tile = workgroup index).
template <bool LB>
__global__ __launch_bounds__(kTileThreads) void k_merge(const uint8_t* __restrict__ packed, int bits,
                                               const uint16_t* __restrict__ fallback, const uint8_t* __restrict__ mask,
                                               const float* __restrict__ scales, int64_t total, int64_t bph,
                                               int64_t n_packed, int64_t n_fallback,
                                               const int64_t* __restrict__ tile_off, uint16_t* __restrict__ out,
                                               uint64_t* __restrict__ status, uint32_t* __restrict__ ticket,
                                               int32_t* __restrict__ err) {
    __shared__ int wcnt[kTile / 64];
    __shared__ int s_t;
    __shared__ int64_t s_off;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int64_t tile = blockIdx.x;
    if constexpr (LB) {
        if (tid == 0) s_t = (int)atomicAdd(ticket, 1u);
        __syncthreads();
        tile = s_t;
    }
    const int64_t t0 = tile * kTile;
    int m[kTileRounds];
    for (int r = 0; r < kTileRounds; r++) {
        int64_t b = t0 + r * kTileThreads + tid;
        m[r] = (b < total && mask[b]) ? 1 : 0;
        unsigned long long bal = __ballot(m[r]);
        if (lane == 0) wcnt[r * (kTileThreads / 64) + wave] = __popcll(bal);
    }
    __syncthreads();
    if constexpr (LB) {
        if (wave == 0) {
            int cnt = 0;
            for (int k = 0; k < kTile / 64; k++) cnt += wcnt[k];
            const int64_t off = tile_lookback(status, tile, cnt, err);
            if (lane == 0) s_off = off;
        }
        __syncthreads();
    }
    const int64_t toff = LB ? s_off : tile_off[tile];
    for (int r = 0; r < kTileRounds; r++) {
        int64_t b = t0 + r * kTileThreads + tid;
        unsigned long long bal = __ballot(m[r]);
        if (b >= total) continue;
        int before = 0;
        for (int k = 0; k < r * (kTileThreads / 64) + wave; k++) before += wcnt[k];
        int64_t rr = toff + before + __popcll(bal & ((1ull << lane) - 1ull));
        // ranks past the rows the caller holds (a mask that selects more rows
        // than packed / fallback have) are clamped: garbage out, never a fault
        if (m[r] && n_packed > 0) {
            rr = rr < n_packed ? rr : n_packed - 1;
            uint64_t w = bits == 4 ? (uint64_t)__builtin_bswap32(reinterpret_cast<const uint32_t*>(packed)[rr])
                                   : load_be(packed + rr * bits, bits);
            float q[8], y[8];
            unpack_word(w, bits, q);
            float s = scales[b / bph];
#pragma unroll
            for (int i = 0; i < 8; i++) y[i] = q[i] * s;
            store8(out, LQ_F16, b, y);
        } else if (!m[r] && n_fallback > 0) {
            int64_t fr = b - rr;
            fr = fr < n_fallback ? fr : n_fallback - 1;
            reinterpret_cast<uint4*>(out)[b] = reinterpret_cast<const uint4*>(fallback)[fr];
        } else {
            reinterpret_cast<uint4*>(out)[b] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
}


// Fixed-rate compression of a (n_heads, bph) batch of vectors in one pass
// (llm/compressed_kv_cache.py compress path of core/compact_storage.py:338-357
// plus the fp16 fallback of the fixed-rate cache): x / scale32[head] -> nearest
// E8 point; in range at `bits` -> its packed word at its rank among the
// in-range vectors, else q * float(scale16[head]) in fp16 at its rank among
// the others; the mask byte; the head of each packed point (optional); tile
// offsets for the merge; the two totals.
//
// SC: the scales are not given but finalised here from the sigma^2 partial
// sums work[head * parts + p] of k_compact_sumsq, for the (at most two, as
// bph >= kTile) heads the tile spans, by the code of k_head_finalize (the
// parts summed in order p = 0, 1, .., lq_scales.h head_scale, the exhaustive
// fast-division check); the tile that holds a head's first vector stores its
// sigma^2 (optional), scale32, scale16 and float(scale16).
struct AutoScales {
    const double* work;
    int parts;
    int scale_bits;
    float* sigma2;
    float* scale32;
    uint16_t* scale16;
    float* scale16f;
};

template <bool SC>
__global__ __launch_bounds__(kTileThreads) void k_compact_encode(
        const void* __restrict__ x, int dtype, int64_t n, int64_t bph, const float* __restrict__ scale32,
        const int32_t* __restrict__ fastdiv, const uint16_t* __restrict__ scale16, int bits,
        uint8_t* __restrict__ mask, uint8_t* __restrict__ packed, uint16_t* __restrict__ fallback,
        int32_t* __restrict__ repr_heads, int64_t* __restrict__ tile_off, int64_t* __restrict__ totals,
        uint64_t* __restrict__ status,
        uint32_t* __restrict__ ticket, int32_t* __restrict__ err, AutoScales as) {
    __shared__ int s_t, s_wcnt[kTile / 64];
    __shared__ int64_t s_excl;
    __shared__ float s_sc[2], s_sf[2];
    __shared__ int s_fd[2], s_bad[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) s_t = (int)atomicAdd(ticket, 1u);
    __syncthreads();
    const int64_t t = s_t;
    const int64_t ntiles = (n + kTile - 1) / kTile;
    int64_t h0 = 0;
    if (SC) {
        const int64_t first = t * kTile, last = (first + kTile < n ? first + kTile : n) - 1;
        h0 = first / bph;
        const int nhd = (int)(last / bph - h0) + 1;   // 1 or 2
        if (wave < nhd) {
            const int64_t h = h0 + wave;
            const double* wp = as.work + h * as.parts;
            double acc = 0.0;
            for (int p0 = 0; p0 < as.parts; p0 += 64) {
                const double v = p0 + lane < as.parts ? wp[p0 + lane] : 0.0;
                const int m = as.parts - p0 < 64 ? as.parts - p0 : 64;
                const uint64_t vb = __builtin_bit_cast(uint64_t, v);
                const int lo = (int)(uint32_t)vb, hi = (int)(uint32_t)(vb >> 32);
                for (int i = 0; i < m; i++) {
                    const uint64_t b = (uint64_t)(uint32_t)__builtin_amdgcn_readlane(lo, i) |
                                       ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, i) << 32);
                    acc += __builtin_bit_cast(double, b);
                }
            }
            if (lane == 0) {
                float s2;
                const float s = head_scale(acc, bph * 8, as.scale_bits, &s2);
                const uint16_t s16 = f2h(s);
                s_sc[wave] = s;
                s_sf[wave] = h2f(s16);
                if (h * bph >= first) {   // the head starts in this tile
                    if (as.sigma2) as.sigma2[h] = s2;
                    as.scale32[h] = s;
                    as.scale16[h] = s16;
                    as.scale16f[h] = h2f(s16);
                }
            }
        }
        __syncthreads();
        for (int k = 0; k < nhd; k++) {
            const int32_t f = dtype == LQ_F16 ? fastdiv_word(s_sc[k], &s_bad[k]) : 0;
            if (tid == 0) s_fd[k] = f;
        }
        __syncthreads();
    }
    const int R = 1 << (bits - 1);
    uint64_t word[kTileRounds];
    float y[kTileRounds][8];
    int m[kTileRounds];
#pragma unroll
    for (int r = 0; r < kTileRounds; r++) {
        const int64_t v = t * kTile + r * kTileThreads + tid;
        m[r] = 0;
        word[r] = 0;
        if (v < n) {
            const int64_t h = v / bph;
            const float s = SC ? s_sc[h - h0] : scale32[h];
            const int32_t fw = SC ? s_fd[h - h0] : fastdiv[h];
            const bool fast = fw != 0;
            const float rs = __int_as_float(fw);   // RN(1 / s) when fast
            float xv[8], tq[8], ic[8];
            load8(x, dtype, v, xv);
#pragma unroll
            for (int i = 0; i < 8; i++) tq[i] = div_scaled(xv[i], s, rs, fast);
            const int c = e8_nearest_fast(tq, ic, [&](float tt[8]) {
                float xx[8];
                load8(x, dtype, v, xx);
#pragma unroll
                for (int i = 0; i < 8; i++) tt[i] = div_scaled(xx[i], s, rs, fast);
            });
            bool in = true;
            uint64_t w = (uint64_t)c;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int ci = (int)ic[i];
                in = in && ci >= -R && ci <= R - 1;
                const uint64_t u = (uint64_t)(uint32_t)(ci + R) & ((1ull << bits) - 1ull);
                w = i < 7 ? (w << bits) | u : (w << (bits - 1)) | (u >> 1);
            }
            m[r] = in ? 1 : 0;
            word[r] = w;
            const float sf = SC ? s_sf[h - h0] : h2f(scale16[h]), off = c ? 0.5f : 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) y[r][i] = (ic[i] + off) * sf;
        }
        const unsigned long long bal = __ballot(m[r]);
        if (lane == 0) s_wcnt[r * (kTileThreads / 64) + wave] = __popcll(bal);
    }
    __syncthreads();
    if (wave == 0) {
        int cnt = 0;
        for (int k = 0; k < kTile / 64; k++) cnt += s_wcnt[k];
        const int64_t excl = tile_lookback(status, t, cnt, err);
        if (lane == 0) {
            s_excl = excl;
            tile_off[t] = excl;
            if (t == ntiles - 1) {
                totals[0] = excl + cnt;
                totals[1] = n - (excl + cnt);
            }
        }
    }
    __syncthreads();
    const int64_t excl = s_excl;
#pragma unroll
    for (int r = 0; r < kTileRounds; r++) {
        const int64_t v = t * kTile + r * kTileThreads + tid;
        const unsigned long long bal = __ballot(m[r]);
        if (v >= n) continue;
        int before = 0;
        for (int k = 0; k < r * (kTileThreads / 64) + wave; k++) before += s_wcnt[k];
        const int64_t rr = excl + before + __popcll(bal & ((1ull << lane) - 1ull));
        mask[v] = (uint8_t)m[r];
        if (m[r]) {
            if (repr_heads) repr_heads[rr] = (int32_t)(v / bph);
            if (bits == 4) {
                reinterpret_cast<uint32_t*>(packed)[rr] = __builtin_bswap32((uint32_t)word[r]);
            } else {
                uint64_t w = word[r];
                for (int b = bits - 1; b >= 0; b--) { packed[rr * bits + b] = (uint8_t)(w & 0xff); w >>= 8; }
            }
        } else {
            store8(fallback, LQ_F16, v - rr, y[r]);
        }
    }
}

}  // namespace

extern "C" {

int lq_unpack_compact(const uint8_t* d_packed, int bits, int64_t n, const float* d_scales, int64_t n_scales,
                      const int32_t* d_head_idx, uint16_t* d_out, hipStream_t s) {
    if (bits < 3 || bits > 5 || n < 0 || n_scales <= 0) return LQ_ERR_ARG;
    if (n == 0) return LQ_OK;
    hipLaunchKernelGGL(k_unpack, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_packed, bits, n, d_scales,
                       n_scales, d_head_idx, d_out);
    return launch_status();
}

int lq_pack_compact(const float* d_q, int bits, int64_t n, uint8_t* d_packed, int32_t* d_ok, hipStream_t s) {
    if (bits < 3 || bits > 5 || n < 0) return LQ_ERR_ARG;
    if (n == 0) return LQ_OK;
    hipLaunchKernelGGL(k_pack, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_q, bits, n, d_packed, d_ok);
    return launch_status();
}

int64_t lq_merge_workspace(int64_t total_blocks) {
    if (total_blocks < 0) return -1;
    return ((total_blocks + kTile - 1) / kTile + 2) * 8;   // tile status words, ticket counter, error flag
}

int lq_fused_merge(const uint8_t* d_packed, int64_t n_packed, int bits, const uint16_t* d_fallback, int64_t n_fallback,
                   const uint8_t* d_mask, const float* d_scales, int64_t total_blocks, int64_t bph, void* d_work,
                   uint16_t* d_out, hipStream_t s) {
    if (bits < 3 || bits > 5 || total_blocks < 0 || bph <= 0 || n_packed < 0 || n_fallback < 0) return LQ_ERR_ARG;
    if (total_blocks == 0) return LQ_OK;
    const int64_t tiles = (total_blocks + kTile - 1) / kTile;
    uint64_t* status = reinterpret_cast<uint64_t*>(d_work);
    uint32_t* ticket = reinterpret_cast<uint32_t*>(status + tiles);
    int32_t* err = reinterpret_cast<int32_t*>(status + tiles + 1);
    hipLaunchKernelGGL(k_zero64, dim3((unsigned)((tiles + 2 + 255) / 256)), dim3(256), 0, s, status, tiles + 2,
                       (int64_t*)nullptr);
    hipLaunchKernelGGL(k_merge<true>, dim3((unsigned)tiles), dim3(kTileThreads), 0, s, d_packed, bits, d_fallback, d_mask,
                       d_scales, total_blocks, bph, n_packed, n_fallback, nullptr, d_out, status, ticket, err);
    return launch_status();
}

int64_t lq_compact_encode_workspace(int64_t n) {
    if (n < 0) return -1;
    return ((n + kTile - 1) / kTile + 1) * 8;   // tile status words, then the ticket counter
}

int lq_compact_encode(const void* d_x, int dtype, int64_t n_heads, int64_t bph, const float* d_scale32,
                      const int32_t* d_fastdiv, const uint16_t* d_scale16, int bits, uint8_t* d_mask,
                      uint8_t* d_packed, uint16_t* d_fallback, int32_t* d_repr_heads, int64_t* d_tile_off,
                      int64_t* d_totals, void* d_work, hipStream_t s) {
    if (bits < 3 || bits > 5 || n_heads <= 0 || bph <= 0 || dtype < 0 || dtype > 2) return LQ_ERR_ARG;
    if (!d_x || !d_scale32 || !d_fastdiv || !d_scale16 || !d_mask || !d_packed || !d_fallback || !d_tile_off ||
        !d_totals || !d_work)
        return LQ_ERR_ARG;
    const int64_t n = n_heads * bph;
    const int64_t tiles = (n + kTile - 1) / kTile;
    uint64_t* status = reinterpret_cast<uint64_t*>(d_work);
    uint32_t* ticket = reinterpret_cast<uint32_t*>(status + tiles);
    int32_t* err = reinterpret_cast<int32_t*>(d_totals + 2);   // read back with the totals
    hipLaunchKernelGGL(k_zero64, dim3((unsigned)((tiles + 1 + 255) / 256)), dim3(256), 0, s, status, tiles + 1,
                       d_totals + 2);
    hipLaunchKernelGGL(k_compact_encode<false>, dim3((unsigned)tiles), dim3(kTileThreads), 0, s, d_x, dtype, n, bph,
                       d_scale32, d_fastdiv, d_scale16, bits, d_mask, d_packed, d_fallback, d_repr_heads, d_tile_off,
                       d_totals, status, ticket, err, AutoScales{});
    return launch_status();
}

int64_t lq_compact_encode_scaled_workspace(int64_t n_heads, int64_t bph) {
    if (n_heads <= 0 || bph <= 0) return -1;
    const int parts = head_parts(n_heads, bph);
    return n_heads * parts * 8 + lq_compact_encode_workspace(n_heads * bph);
}

int lq_compact_encode_scaled(const void* d_x, int dtype, int64_t n_heads, int64_t bph, int scale_bits, int bits,
                             float* d_sigma2, float* d_scale32, uint16_t* d_scale16, float* d_scale16f,
                             uint8_t* d_mask, uint8_t* d_packed, uint16_t* d_fallback, int32_t* d_repr_heads,
                             int64_t* d_tile_off, int64_t* d_totals, void* d_work, hipStream_t s) {
    if (bits < 3 || bits > 5 || scale_bits < 1 || scale_bits > 16 || n_heads <= 0 || bph < kTile || dtype < 0 ||
        dtype > 2)
        return LQ_ERR_ARG;
    if (!d_x || !d_scale32 || !d_scale16 || !d_scale16f || !d_mask || !d_packed || !d_fallback || !d_tile_off ||
        !d_totals || !d_work)
        return LQ_ERR_ARG;
    const int64_t n = n_heads * bph;
    const int64_t tiles = (n + kTile - 1) / kTile;
    const int parts = head_parts(n_heads, bph);
    double* partial = reinterpret_cast<double*>(d_work);
    uint64_t* status = reinterpret_cast<uint64_t*>(partial + n_heads * parts);
    uint32_t* ticket = reinterpret_cast<uint32_t*>(status + tiles);
    int32_t* err = reinterpret_cast<int32_t*>(d_totals + 2);   // read back with the totals
    hipLaunchKernelGGL(k_compact_sumsq, dim3((unsigned)n_heads, parts), dim3(256), 0, s, d_x, dtype, bph, parts,
                       partial, status, tiles + 1, d_totals + 2);
    const AutoScales as{partial, parts, scale_bits, d_sigma2, d_scale32, d_scale16, d_scale16f};
    hipLaunchKernelGGL(k_compact_encode<true>, dim3((unsigned)tiles), dim3(kTileThreads), 0, s, d_x, dtype, n, bph,
                       (const float*)nullptr, (const int32_t*)nullptr, (const uint16_t*)nullptr, bits, d_mask,
                       d_packed, d_fallback, d_repr_heads, d_tile_off, d_totals, status, ticket, err, as);
    return launch_status();
}

int lq_compact_merge(const uint8_t* d_packed, int64_t n_packed, int bits, const uint16_t* d_fallback,
                     int64_t n_fallback, const uint8_t* d_mask, const float* d_scales, int64_t total_blocks,
                     int64_t bph, const int64_t* d_tile_off, uint16_t* d_out, hipStream_t s) {
    if (bits < 3 || bits > 5 || total_blocks < 0 || bph <= 0 || n_packed < 0 || n_fallback < 0 || !d_tile_off)
        return LQ_ERR_ARG;
    if (total_blocks == 0) return LQ_OK;
    const int64_t tiles = (total_blocks + kTile - 1) / kTile;
    hipLaunchKernelGGL(k_merge<false>, dim3((unsigned)tiles), dim3(kTileThreads), 0, s, d_packed, bits, d_fallback, d_mask,
                       d_scales, total_blocks, bph, n_packed, n_fallback, d_tile_off, d_out, nullptr, nullptr, nullptr);
    return launch_status();
}

int lq_version(void) { return 10000; }

int lq_hip_runtime_version(void) {
    int v = 0;
    if (hipRuntimeGetVersion(&v) != hipSuccess) return -1;
    return v;
}

const char* lq_status_string(int code) {
    switch (code) {
        case LQ_OK: return "ok";
        case LQ_ERR_ARG: return "invalid argument";
        case LQ_ERR_LAUNCH: return "kernel launch failed";
        case LQ_ERR_ALPHABET: return "rANS alphabet larger than L = 1024";
        case LQ_ERR_RANGE: return "lattice symbol outside int8";
        case LQ_ERR_SCRATCH: return "request larger than the static scratch array";
        default: return "unknown status";
    }
}

}  // extern "C"
