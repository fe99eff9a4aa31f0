// rANS kernels for gfx950: table construction, block-parallel encode of the
// reference's bit-wise streams, bitstream assembly and checkpointed decode.
//
// Stream format (reference core/gpu_ans.py:105-139): L = 1024, state in
// [1024, 2048), one renormalisation bit at a time; the encoder runs over the
// symbols in reverse and the emitted bit list is reversed and packed LSB-first
// into uint32 words, followed by one zero word.
//
// Parallel encode: the state after a symbol depends only on the high bits of
// the state before it, so encoder trajectories from different starting states
// merge.  A lane that owns block g tracks the interval [lo, hi] of every state
// that can enter it, starting from the full range a few symbols earlier (in
// encode order); once lo == hi the entering state is known exactly, whatever
// the true history.  If the interval has not collapsed the window grows, up to
// the end of the stream where the state is exactly L.  Results are therefore
// exact, and identical to a serial encode.
#include <climits>

#include "lq_argsort.h"
#include "lq_decode.h"

using namespace lq;

namespace {

inline int launch_status() { return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_LAUNCH; }

// Compute units of the current device (cached per device; 256 on MI355X).
inline int64_t device_cus() {
    static int64_t cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cache[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

// The table code runs on a cooperative group: a whole workgroup (one stream
// per workgroup), or one wave (one stream per wave, wave-synchronous: no
// workgroup barrier).  G::tid / G::size / G::sync are the group's lane, size
// and LDS barrier.
struct BlockGroup {
    static __device__ __forceinline__ int tid() { return (int)threadIdx.x; }
    static __device__ __forceinline__ int size() { return (int)blockDim.x; }
    static __device__ __forceinline__ void sync() { __syncthreads(); }
    static constexpr bool kWave = false;
};
struct WaveGroup {
    static __device__ __forceinline__ int tid() { return (int)(threadIdx.x & 63); }
    static __device__ __forceinline__ int size() { return 64; }
    static __device__ __forceinline__ void sync() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    static constexpr bool kWave = true;
};

// Block-wide sum of v (G::size() multiple of 64, <= 1024).
template <typename G>
__device__ int64_t block_sum(int64_t v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if constexpr (G::kWave) return v;
    __shared__ int64_t part[16];
    G::sync();
    if ((G::tid() & 63) == 0) part[G::tid() >> 6] = v;
    G::sync();
    int64_t s = 0;
    for (int w = 0; w < (int)(G::size() >> 6); w++) s += part[w];
    return s;
}

// Block-wide maximum of v (G::size() multiple of 64, <= 1024).
template <typename G>
__device__ int64_t block_max(int64_t v) {
    for (int o = 32; o > 0; o >>= 1) {
        const int64_t u = __shfl_xor(v, o, 64);
        v = u > v ? u : v;
    }
    if constexpr (G::kWave) return v;
    __shared__ int64_t part[16];
    G::sync();
    if ((G::tid() & 63) == 0) part[G::tid() >> 6] = v;
    G::sync();
    int64_t m = part[0];
    for (int w = 1; w < (int)(G::size() >> 6); w++) m = part[w] > m ? part[w] : m;
    return m;
}

// Bitonic sort of c[0 .. N) ascending (N a power of two, c padded with
// UINT64_MAX past the live entries).
template <typename G>
__device__ void bitonic_sort_u64(uint64_t* c, int N) {
    for (int k = 2; k <= N; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int t = G::tid(); t < N / 2; t += G::size()) {
                const int i = 2 * t - (t & (j - 1));   // low index of the pair: bit j clear
                const int l = i + j;
                const bool up = (i & k) == 0;
                const uint64_t x = c[i], y = c[l];
                if ((x > y) == up) { c[i] = y; c[l] = x; }
            }
            G::sync();
        }
    }
}

// adjust_pass for alphabets above 256 symbols: the members of the set
// (the first rem entries of the argsort order) that do not depend on the tie
// order, from one bitonic sort of composite (key, index) keys instead of
// per-entry rank counts.  At most one tie group straddles the cut at sorted
// position rem: the one holding positions rem - 1 and rem.  Returns (group
// uniform) whether a different subset of that group would change a frequency.
template <typename G>
__device__ bool adjust_pass_sorted(int n, const int32_t* freqs, int diff, int full, int rem, const int64_t* kk,
                                   int16_t* a, int8_t* inset, uint64_t* sk) {
    int N = 512;
    while (N < n) N <<= 1;
    for (int i = G::tid(); i < N; i += G::size())   // kk in [-(2^32 - 1), 0]: biased key in 33 bits
        sk[i] = i < n ? (((uint64_t)(kk[i] + (int64_t)4294967296LL)) << 11) | (uint64_t)i : ~0ull;
    G::sync();
    bitonic_sort_u64<G>(sk, N);
    for (int p = G::tid(); p < n; p += G::size()) {
        const int i = (int)(sk[p] & 2047u);
        a[p] = (int16_t)i;
        inset[i] = p < rem ? 1 : 0;
    }
    G::sync();
    int matters = 0;
    if (rem > 0 && rem < n && (sk[rem - 1] >> 11) == (sk[rem] >> 11)) {   // uniform
        const uint64_t kstar = sk[rem] >> 11;
        for (int p = G::tid(); p < n; p += G::size())
            if ((sk[p] >> 11) == kstar && (diff > 0 || freqs[a[p]] - full > 1)) matters = 1;
    }
    return block_sum<G>(matters) != 0;
}

// One pass of the build_rans_table adjustment loop (core/gpu_ans.py:73-84)
// with m = |diff|: j = 0 .. m-1 visits order[j % n], i.e. every entry
// `full` = m / n times plus the first rem = m % n entries of the argsort order
// once more; an increment adds its visits, a decrement leaves
// max(f - visits, 1).  The argsort tie order only matters for the tie group
// straddling position rem, and only if a different subset of that group would
// change a frequency; numpy's argsort (np_argsort) runs only then.
template <typename G>
__device__ void adjust_pass(const int64_t* counts, int n, int32_t* freqs, int diff, int16_t* a, int64_t* kk,
                            int8_t* inset, NpScratch* ns, uint64_t* sk) {
    const int m = diff > 0 ? diff : -diff;
    const int full = m / n, rem = m % n;
    for (int i = G::tid(); i < n; i += G::size()) kk[i] = diff > 0 ? -counts[i] : -(int64_t)freqs[i];
    G::sync();
    bool matters;
    if (n > 256 && sk) {
        matters = adjust_pass_sorted<G>(n, freqs, diff, full, rem, kk, a, inset, sk);
    } else {
        int mt = 0;
        for (int i = G::tid(); i < n; i += G::size()) {
            const int64_t ki = kk[i];
            int lt = 0, eq = 0;
            for (int j = 0; j < n; j++) { lt += kk[j] < ki; eq += kk[j] == ki; }
            const int8_t in = lt + eq <= rem ? 1 : (lt >= rem ? 0 : 2);
            inset[i] = in;
            if (in == 2 && (diff > 0 || freqs[i] - full > 1)) mt = 1;
        }
        matters = block_sum<G>(mt) != 0;
    }
    if (matters) {
        if (n <= 256) {   // numpy's network directly (np_argsort's first and only frame)
            for (int i = G::tid(); i < n; i += G::size()) { ns->k[i] = kk[i]; ns->a[i] = (int16_t)i; }
            G::sync();
            np_net_sort<G>(ns->k, ns->a, n);
            for (int p = G::tid(); p < n; p += G::size()) inset[ns->a[p]] = p < rem ? 1 : 0;
        } else {
            np_argsort<G>(kk, a, n, ns);
            for (int p = G::tid(); p < n; p += G::size()) inset[a[p]] = p < rem ? 1 : 0;
        }
        G::sync();
    }
    for (int i = G::tid(); i < n; i += G::size()) {
        const int v = full + (inset[i] == 1 ? 1 : 0);
        const int f = freqs[i];
        freqs[i] = diff > 0 ? f + v : (f - v > 1 ? f - v : 1);
    }
    G::sync();
}

// build_rans_table normalisation (core/gpu_ans.py:62-86) on LDS arrays:
// counts[n] (int64) in, freqs[n] (int32) out; a, kk, inset: n entries;
// ns: argsort scratch; sk (optional, alphabets above 256): 2048 entries.
//
// An increment pass always reaches sum == L.  In the decrement branch the
// excess is below n (only the max(., 1) bumps exceed L), so a pass whose
// excess covers all G entries with f > 1 decrements exactly those, whatever
// the order; such passes are counted in closed form and only the last,
// partial pass (excess < G) goes through adjust_pass.  The number t of full
// passes is the least t with G_t = 0 or C(t + 1) > excess, where
// G_t = #{f_i - t > 1} and C(t) = G_0 + .. + G_(t-1) = sum_i min(t, f_i - 1)
// is nondecreasing: a binary search over t in [0, max f - 1], not one pass
// per t (a single dominant symbol makes t as large as the excess).
template <typename G>
__device__ void normalise(const int64_t* counts, int n, int32_t* freqs, int16_t* a, int64_t* kk, int8_t* inset,
                          NpScratch* ns, uint64_t* sk = nullptr) {
    int64_t tl = 0;
    for (int i = G::tid(); i < n; i += G::size()) tl += counts[i];
    const int64_t total = block_sum<G>(tl);
    int64_t fl = 0;
    for (int i = G::tid(); i < n; i += G::size()) {
        int32_t f = 1;
        if (total != 0) {
            double q = (double)counts[i] / (double)total * (double)kL;   // (counts / total * L)
            int32_t t = (int32_t)q;                                       // .astype(int32)
            f = t < 1 ? 1 : t;
        }
        freqs[i] = f;
        fl += f;
    }
    const int diff = (int)(kL - block_sum<G>(fl));
    if (diff > 0) {
        adjust_pass<G>(counts, n, freqs, diff, a, kk, inset, ns, sk);
    } else if (diff < 0) {
        const int excess0 = -diff;
        int64_t fm = 0;
        for (int i = G::tid(); i < n; i += G::size()) fm = freqs[i] > fm ? freqs[i] : fm;
        const int fmax = (int)block_max<G>(fm);
        auto C = [&](int tt) {   // passes 0 .. tt-1 decrement sum_i min(tt, f_i - 1) entries in total
            int64_t c = 0;
            for (int i = G::tid(); i < n; i += G::size()) {
                const int r = freqs[i] - 1;
                c += r < tt ? r : tt;
            }
            return block_sum<G>(c);
        };
        int lo = 0, hi = fmax - 1 > 0 ? fmax - 1 : 0;   // t = fmax - 1 has G_t = 0
        while (lo < hi) {   // least t in [0, hi) with C(t + 1) > excess, else hi
            const int mid = (lo + hi) >> 1;
            if (C(mid + 1) > excess0) hi = mid; else lo = mid + 1;
        }
        const int t = lo;
        const int excess = (int)(excess0 - C(t));
        for (int i = G::tid(); i < n; i += G::size()) freqs[i] = freqs[i] - t > 1 ? freqs[i] - t : 1;
        G::sync();
        if (excess > 0) adjust_pass<G>(counts, n, freqs, -excess, a, kk, inset, ns, sk);
    }
}

// Inclusive scan of v over the block (G::size() <= 1024, multiple of 64).
template <typename G>
__device__ int block_incl_scan(int v) {
    const int lane = G::tid() & 63, w = G::tid() >> 6;
    for (int o = 1; o < 64; o <<= 1) {
        int t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    if constexpr (G::kWave) return v;
    __shared__ int wsum[16];
    G::sync();
    if (lane == 63) wsum[w] = v;
    G::sync();
    for (int i = 0; i < w; i++) v += wsum[i];
    return v;
}

// out[i] = in[0] + .. + in[i-1] for i <= n (block-cooperative, any n).
template <typename G>
__device__ void exclusive_scan_array(const int32_t* in, int n, int32_t* out) {
    if constexpr (G::kWave) {   // the carry stays in registers (uniform over the wave)
        int carry = 0;
        for (int b = 0; b < n; b += 64) {
            const int i = b + G::tid();
            const int v = i < n ? in[i] : 0;
            const int incl = block_incl_scan<G>(v);
            if (i < n) out[i] = carry + incl - v;
            carry += __shfl(incl, 63, 64);
        }
        if (G::tid() == 0) out[n] = carry;
        G::sync();
        return;
    }
    __shared__ int carry;
    if (G::tid() == 0) carry = 0;
    G::sync();
    for (int b = 0; b < n; b += G::size()) {
        int i = b + G::tid();
        int v = i < n ? in[i] : 0;
        int incl = block_incl_scan<G>(v);
        int c = carry;
        if (i < n) out[i] = c + incl - v;
        G::sync();
        if (G::tid() == G::size() - 1) carry = c + incl;
        G::sync();
    }
    if (G::tid() == 0) out[n] = carry;
    G::sync();
}

// ------------------------------------------------------------ chunk tables --

// WIDE = false: hist holds 16 x 256 int8-symbol bins (value + 128).
// WIDE = true:  hist holds 16 x 1024 bins from the stream's min (minmax).
template <bool WIDE>
__global__ __launch_bounds__(256) void k_chunk_tables(const uint32_t* __restrict__ hist, const int32_t* __restrict__ minmax,
                                                      lq_table* __restrict__ tables, int32_t* __restrict__ status) {
    __shared__ int64_t counts[LQ_MAXSYM];
    __shared__ int32_t freqs[LQ_MAXSYM];
    __shared__ NpScratch ns;
    __shared__ int16_t perm[LQ_MAXSYM];
    __shared__ uint32_t h[256];
    __shared__ int s_min, s_max, s_st;
    __shared__ uint32_t s_tot;
    const int64_t sid = blockIdx.x;   // chunk * 16 + stream
    const int tid = threadIdx.x;
    lq_table* T = tables + sid;
    int lo, n;
    if constexpr (!WIDE) {
        h[tid] = hist[sid * 256 + tid];
        if (tid == 0) { s_min = 256; s_max = -1; s_tot = 0; s_st = 0; }
        __syncthreads();
        if (h[tid]) { atomicMin(&s_min, tid); atomicMax(&s_max, tid); atomicAdd(&s_tot, h[tid]); }
        __syncthreads();
        if (s_max < 0) {
            if (tid == 0) { T->lo = 0; T->n_sym = 0; T->n_symbols = 0; T->status = 0; }
            return;
        }
        lo = s_min - 128 - 2;
        n = s_max - s_min + 5;
        for (int i = tid; i < n; i += 256) {
            int b = lo + i + 128;
            counts[i] = (b >= 0 && b < 256) ? (int64_t)h[b] : 0;
        }
    } else {
        const int mn = minmax[sid * 2], mx = minmax[sid * 2 + 1];
        if (mx == INT_MIN) {   // absent stream (empty coset)
            if (tid == 0) { T->lo = 0; T->n_sym = 0; T->n_symbols = 0; T->status = 0; }
            return;
        }
        lo = mn - 2;
        n = mx - mn + 5;
        if (n > kL) {   // the reference's normalisation never terminates here
            if (tid == 0) {
                T->lo = lo; T->n_sym = 0; T->n_symbols = 0; T->status = LQ_ST_ALPHABET;
                atomicOr(status + sid / LQ_STREAMS, LQ_ST_ALPHABET);
            }
            return;
        }
        if (tid == 0) { s_tot = 0; s_st = 0; }
        __syncthreads();
        uint32_t tl = 0;
        for (int i = tid; i < n; i += 256) {
            const uint32_t c = (i >= 2 && i - 2 < kL) ? hist[sid * kL + i - 2] : 0u;
            counts[i] = c;
            tl += c;
        }
        atomicAdd(&s_tot, tl);
    }
    __syncthreads();
    __shared__ int64_t kk[LQ_MAXSYM];
    __shared__ int8_t inset[LQ_MAXSYM];
    __shared__ uint64_t sk[WIDE ? 2048 : 1];   // wide alphabets: composite sort keys
    normalise<BlockGroup>(counts, n, freqs, perm, kk, inset, &ns, WIDE ? sk : nullptr);
    __shared__ int32_t cum[LQ_MAXSYM + 1];
    exclusive_scan_array<BlockGroup>(freqs, n, cum);
    for (int i = tid; i < n; i += 256) T->enc[i] = enc_pack((uint32_t)freqs[i], (uint32_t)cum[i]);
    if (tid == 0) {
        T->lo = lo;
        T->n_sym = n;
        T->n_symbols = (int32_t)s_tot;
        T->status = s_st;
        if (s_st) atomicOr(status + sid / LQ_STREAMS, s_st);
    }
}

// int8 path: one wave per stream, kTabWaves streams per workgroup; the
// stream's table built wave-synchronously (WaveGroup) in its own LDS arrays,
// with the same normalisation and tie order as k_chunk_tables<false>.
constexpr int kTabWaves = 4;
constexpr int kCap8 = 264;   // range(min - 2, max + 2) of int8 values: at most 260 symbols

__global__ __launch_bounds__(64 * kTabWaves) void k_chunk_tables_wave(const uint32_t* __restrict__ hist,
                                                                      int64_t n_streams, lq_table* __restrict__ tables,
                                                                      int32_t* __restrict__ status) {
    __shared__ int64_t counts[kTabWaves][kCap8];
    __shared__ int32_t freqs[kTabWaves][kCap8];
    __shared__ NpScratch ns[kTabWaves];
    __shared__ int16_t perm[kTabWaves][kCap8];
    __shared__ int64_t kk[kTabWaves][kCap8];
    __shared__ int8_t inset[kTabWaves][kCap8];
    __shared__ int32_t cum[kTabWaves][kCap8 + 1];
    __shared__ int s_st[kTabWaves];
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = (int)(threadIdx.x & 63);
    const int64_t sid = (int64_t)blockIdx.x * kTabWaves + w;
    if (sid >= n_streams) return;   // wave-uniform; no workgroup barrier below
    lq_table* T = tables + sid;
    const uint32_t* hs = hist + sid * 256;
    uint32_t hv[4];
    int mn = 256, mx = -1;
    uint32_t tl = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int b = lane + 64 * j;
        hv[j] = hs[b];
        if (hv[j]) {
            mn = b < mn ? b : mn;
            mx = b > mx ? b : mx;
            tl += hv[j];
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const int a = __shfl_xor(mn, o, 64), c = __shfl_xor(mx, o, 64);
        mn = a < mn ? a : mn;
        mx = c > mx ? c : mx;
        tl += __shfl_xor(tl, o, 64);
    }
    if (mx < 0) {   // absent stream (empty coset)
        if (lane == 0) { T->lo = 0; T->n_sym = 0; T->n_symbols = 0; T->status = 0; }
        return;
    }
    const int lo = mn - 128 - 2, n = mx - mn + 5;
    for (int i = lane; i < n; i += 64) {
        const int b = lo + i + 128;
        counts[w][i] = (b >= 0 && b < 256) ? (int64_t)hs[b] : 0;
    }
    if (lane == 0) s_st[w] = 0;
    WaveGroup::sync();
    normalise<WaveGroup>(counts[w], n, freqs[w], perm[w], kk[w], inset[w], &ns[w]);
    exclusive_scan_array<WaveGroup>(freqs[w], n, cum[w]);
    for (int i = lane; i < n; i += 64) T->enc[i] = enc_pack((uint32_t)freqs[w][i], (uint32_t)cum[w][i]);
    if (lane == 0) {
        const int st = s_st[w];
        T->lo = lo;
        T->n_sym = n;
        T->n_symbols = (int32_t)tl;
        T->status = st;
        if (st) atomicOr(status + sid / LQ_STREAMS, st);
    }
}

// ------------------------------------------------------------ chunk encode --
//
// Task = (chunk, stream st = coset * 8 + coord, block g), one lane each; a
// 256-thread workgroup holds 16 consecutive blocks x 16 streams of one chunk,
// a wave one coset of 8 blocks, so the 8 lanes of a (block, coset) read the 8
// interleaved columns of that coset one 128-byte line at a time (sym_pos
// layout).

template <typename SymT>
struct Col {
    const SymT* p;   // chunk 0 of the column; chunk k at p + 128 k (elements)
    int n;
};

template <typename SymT>
__device__ __forceinline__ Col<SymT> column(const SymT* sym, const uint32_t* blk_n1, int64_t chunk, int64_t nblk,
                                            int64_t V, int64_t h, int c, int idx) {
    uint32_t n1 = blk_n1[chunk * nblk + h];
    int64_t valid = V - h * kBlk < kBlk ? V - h * kBlk : kBlk;
    int n0 = (int)valid - (int)n1;
    Col<SymT> col;
    col.p = sym + (chunk * nblk + h) * (int64_t)kSymStride + sym_region(c, n0) + 16 * idx;
    col.n = c ? (int)n1 : n0;
    return col;
}

// f(v, b, in) for the column symbols of ranks n-1, n-2, .., 0 (the column's
// 16-symbol chunk k sits at p + 128 k), read with 16-byte loads issued one
// chunk ahead.  b is the symbol's index in its chunk (a compile-time
// constant after unrolling).  Only a column's top chunk can be partial.
// Control flow is wave-uniform: the loop runs while any lane has chunks left,
// takes the unconditional path when every lane holds a full chunk, the same
// path with finished lanes masked off when every lane holds a full chunk or
// none, and otherwise passes a per-lane predicate; f must leave its state
// unchanged when in == false.
template <typename SymT, typename F>
__device__ __forceinline__ void for_each_rev(const SymT* p, int n, F&& f) {
    int k = n > 0 ? (n - 1) >> 4 : -1;   // current chunk
    Chunk16<SymT> cur = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)}, nxt = cur;
    if (k >= 0) cur = gload_chunk(p + 128 * (int64_t)k);
    if (k >= 1) nxt = gload_chunk(p + 128 * (int64_t)(k - 1));
    while (__any(k >= 0)) {
        const int hi_b = k < 0 ? 0 : (n - 16 * k < 16 ? n - 16 * k : 16);
        if (__all(hi_b == 16)) {
#pragma unroll
            for (int b = 15; b >= 0; b--) f(cur.get(b), b, true);
        } else if (__all(hi_b == 16 || hi_b == 0)) {
            // every lane holds a full chunk or has none left (the columns of a
            // wave end at different chunks): the full path, finished lanes
            // masked off
            if (hi_b == 16) {
#pragma unroll
                for (int b = 15; b >= 0; b--) f(cur.get(b), b, true);
            }
        } else {
#pragma unroll
            for (int b = 15; b >= 0; b--) f(cur.get(b), b, b < hi_b);
        }
        k--;
        cur = nxt;
        if (k >= 1) nxt = gload_chunk(p + 128 * (int64_t)(k - 1));
    }
}

struct EncWork {  // offsets into the encode workspace
    int64_t bits, scratch, tiles, total;
};

// Streams longer than kScanTile blocks are scanned in tiles (k_scan_tiles /
// k_scan_top / k_scan_apply, then k_chunk_offsets); shorter ones by one
// workgroup per chunk (k_chunk_scan_offsets).
constexpr int kScanTile = 4096;

__host__ __device__ inline EncWork enc_layout(int64_t n_chunks, int64_t n_vectors) {
    int64_t nblk = (n_vectors + kBlk - 1) / kBlk;
    int64_t tasks = n_chunks * LQ_STREAMS * nblk;
    int64_t n_tiles = nblk > kScanTile ? n_chunks * LQ_STREAMS * ((nblk + kScanTile - 1) / kScanTile) : 0;
    EncWork w;
    w.bits = 0;
    w.scratch = ((tasks * 4 + 255) / 256) * 256;
    w.tiles = w.scratch + tasks * (int64_t)kCapW * 4;
    w.total = w.tiles + n_tiles * 8;
    return w;
}

constexpr int kEncBlocks = 16;   // blocks per encode workgroup (x 16 streams)

// Grid: (block groups, chunks).  The scratch words of a task are collected in
// a 4-word LDS queue per lane and stored as aligned 16-byte pieces.
template <typename SymT>
__global__ __launch_bounds__(256) void k_chunk_encode(const SymT* __restrict__ sym, const uint32_t* __restrict__ blk_n1,
                                                      int64_t nblk, int64_t V, const lq_table* __restrict__ tables,
                                                      uint32_t* __restrict__ blk_bits, uint32_t* __restrict__ scratch,
                                                      uint16_t* __restrict__ blk_state) {
    // odd row stride: the 16 stream tables start in different LDS banks.
    // int8 symbols span at most 260 alphabet entries, all held in LDS.  Wide
    // (int16) alphabets reach L + 4 entries: LDS holds a window of kWin
    // entries per stream around symbol 0 (lattice coordinates centre there),
    // and the rare symbol outside it reads its entry from the table in global
    // memory, so the workgroup's LDS stays that of the int8 encoder.
    constexpr bool kWide = sizeof(SymT) == 2;
    constexpr int kWin = kWide ? 256 : 264;
    __shared__ uint32_t senc[LQ_STREAMS][kWin + 1];
    __shared__ int slo[LQ_STREAMS], snsym[LQ_STREAMS];
    __shared__ uint32_t sq[4][256];   // per-lane queue of scratch words (4: seven workgroups fit a CU's LDS)
    const int tid = threadIdx.x;
    const int64_t chunk = blockIdx.y;
    // wave = one coset of 8 blocks (lanes: block-major, coordinate-minor), so
    // a wave's columns hold one coset's counts and run about equally long
    const int64_t g = (int64_t)blockIdx.x * kEncBlocks + ((tid >> 3) & 15);
    const int st = ((tid >> 7) << 3) | (tid & 7);
    const lq_table* T = tables + chunk * LQ_STREAMS;
    // first alphabet entry of stream s's LDS window
    auto win0 = [&](int s) -> int {
        if constexpr (!kWide) return 0;
        const int n = T[s].n_sym, w = -T[s].lo - kWin / 2;
        return n <= kWin || w <= 0 ? 0 : (w < n - kWin ? w : n - kWin);
    };
    for (int i = tid; i < LQ_STREAMS * kWin; i += 256) {
        const int s = i / kWin, j = i % kWin, w0 = win0(s);
        senc[s][j] = j + w0 < T[s].n_sym ? encx_of(T[s].enc[j + w0]) : 0u;
    }
    if (tid < LQ_STREAMS) { slo[tid] = T[tid].lo + win0(tid); snsym[tid] = T[tid].n_sym; }
    __syncthreads();
    if (g >= nblk) return;
    const int64_t task = (chunk * LQ_STREAMS + st) * nblk + g;
    if (snsym[st] == 0) {  // absent stream (empty coset)
        blk_bits[task] = 0;
        blk_state[task] = (uint16_t)kL;
        return;
    }
    const int c = st >> 3, idx = st & 7;
    const uint32_t* encs = senc[st];
    const int lo_sym = slo[st];   // symbol of the window's first entry (a valid symbol)
    const uint32_t* const genc = T[st].enc;
    const int glo = T[st].lo;
    auto enc = [&](int v) -> uint32_t {   // entry of symbol value v
        const uint32_t j = (uint32_t)(v - lo_sym);
        if constexpr (!kWide) {
            return encs[j];
        } else {
            uint32_t e = encs[j < (uint32_t)kWin ? j : (uint32_t)kWin - 1u];
            if (j >= (uint32_t)kWin) e = encx_of(genc[v - glo]);   // outside the window (rare)
            return e;
        }
    };

    // ---- state entering block g (encode order runs from the stream end down)
    uint32_t x = kL;
    int window = 16;   // symbols after the block; the interval collapses within 16 on typical tables
    for (;;) {
        // top of the window: `window` symbols after block g, or the stream end
        int64_t h = g + 1;
        int need = window;
        while (h < nblk) {
            int nc = column(sym, blk_n1, chunk, nblk, V, h, c, idx).n;
            if (need <= nc) break;
            need -= nc;
            h++;
        }
        const bool exact = h >= nblk;
        uint32_t lo = kL, hi = exact ? (uint32_t)kL : 2u * kL - 1u;
        const int64_t hb = exact ? nblk - 1 : h;
        for (int64_t b = hb; b > g; b--) {
            Col<SymT> col = column(sym, blk_n1, chunk, nblk, V, b, c, idx);
            const int cnt = (b == hb && !exact) ? need : col.n;
            if (lo == hi) {
                uint32_t xx = lo, k;
                for_each_rev(col.p, cnt, [&](int v, int, bool in) {
                    const uint32_t xn = encx_step(xx, enc(in ? v : lo_sym), &k);
                    xx = in ? xn : xx;
                });
                lo = hi = xx;
            } else {
                for_each_rev(col.p, cnt, [&](int v, int, bool in) {
                    uint32_t l2 = lo, h2 = hi;
                    hull_step(l2, h2, enc(in ? v : lo_sym));
                    lo = in ? l2 : lo;
                    hi = in ? h2 : hi;
                });
            }
        }
        if (lo == hi) { x = lo; break; }
        window *= 8;
    }

    // ---- encode block g, bits right-aligned in the task's scratch region
    Col<SymT> col = column(sym, blk_n1, chunk, nblk, V, g, c, idx);
    uint32_t* scr = scratch + task * (int64_t)kCapW;
    // words leave in decreasing address order from kCapW - 1; word j of the
    // current 4-word group waits in LDS at qcol[(3 - j) * 256] (this lane's
    // column, so a wave's writes are contiguous) and the group leaves as one
    // 16-byte store when full
    uint32_t* const qcol = &sq[0][tid];
    int nq = 0, gbase = kCapW - 4, nwords = 0;
    auto push = [&](uint32_t word) {
        qcol[(3 - nq) * 256] = word;
        nwords++;
        if (++nq == 4) {
            *reinterpret_cast<uint4*>(scr + gbase) = make_uint4(qcol[0], qcol[256], qcol[512], qcol[768]);
            gbase -= 4;
            nq = 0;
        }
    };
    // Bit accumulator (ahi:alo): the emitted bits sit at the top, newest
    // highest; a symbol's group (the k low bits of xin, bit k - 1 first in the
    // final stream) enters by one funnel shift of (xin:ahi:alo) right by k, two
    // v_alignbit (k <= 10; k = 0 leaves all three in place).  Below the bits a
    // single 1 (the sentinel) marks their end, so no bit count is kept: 32 or
    // more bits are held exactly when the low word is nonzero.  The oldest 32
    // bits then leave as one word, bit-reversed so that the oldest bit is the
    // word's most significant, as the stream order wants.
    uint32_t ahi = 0x80000000u, alo = 0u;
    auto take_word = [&]() {   // needs alo != 0
        const uint32_t s = (uint32_t)__builtin_ctz(alo);   // sentinel position
        const uint32_t raw = (uint32_t)((((uint64_t)ahi << 32) | alo) >> (s + 1u));
        push(__builtin_bitreverse32(raw));
        ahi = ((ahi >> s) | 1u) << s;   // sentinel moves up 32 bits (to bit s of the high word)
        alo = 0u;
    };
    for_each_rev(col.p, col.n, [&](int v, int b, bool in) {
        uint32_t k;
        const uint32_t xin = x;
        const uint32_t xn = encx_step(xin, enc(in ? v : lo_sym), &k);
        k = in ? k : 0u;
        x = in ? xn : xin;
        alo = __builtin_amdgcn_alignbit(ahi, alo, k);
        ahi = __builtin_amdgcn_alignbit(xin, ahi, k);
        // at most 3 symbols (<= 30 bits) since the last check: <= 61 bits and the sentinel
        if (b % 3 == 0 && alo != 0u) take_word();
    });
    if (alo != 0u) take_word();   // the range may end between check points
    // fewer than 32 bits left: the sentinel is in the high word
    const uint32_t nacc = 31u - (uint32_t)__builtin_ctz(ahi);
    const uint32_t total = 32u * (uint32_t)nwords + nacc;
    if (nacc) push(__builtin_bitreverse32(ahi >> (32u - nacc)));
    if (nq) {   // the last, partial group: its words sit in the top nq slots
        *reinterpret_cast<uint4*>(scr + gbase) = make_uint4(qcol[0], qcol[256], qcol[512], qcol[768]);
    }
    blk_bits[task] = total;
    blk_state[task] = (uint16_t)x;
}

// Short streams (nblk <= kScanTile), one workgroup per chunk, wave w = stream
// w: exclusive prefix of the block bit counts (64 blocks per round, a wave
// scan plus the running carry), n_bits and final state; then the chunk's word
// offsets (n_words + 1 words per present stream) and total.  Replaces
// k_chunk_scan + k_chunk_offsets for such batches.
constexpr int kScanRounds = 32;   // rounds of 64 blocks whose loads are in flight together

// Inclusive scan over the 64 lanes of a wave in DPP moves: Hillis-Steele
// within each 16-lane row (row_shr 1, 2, 4, 8; lanes shifted in from outside
// the row read 0), then row 0's last lane added to row 1 and row 2's to row 3
// (row_bcast:15), then lane 31 added to rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
    int v = (int)x;
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1 and 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2 and 3
    return (uint32_t)v;
}

__global__ __launch_bounds__(1024) void k_chunk_scan_offsets(const uint32_t* __restrict__ blk_bits,
                                                             const uint16_t* __restrict__ blk_state,
                                                             const lq_table* __restrict__ tables, int64_t nblk,
                                                             uint32_t* __restrict__ blk_off,
                                                             int64_t* __restrict__ stream_nbits,
                                                             int32_t* __restrict__ stream_state,
                                                             int64_t* __restrict__ stream_woff,
                                                             int64_t* __restrict__ chunk_words) {
    __shared__ int64_t s_nbits[LQ_STREAMS];
    __shared__ int s_present[LQ_STREAMS];
    const int64_t c = blockIdx.x;
    const int lane = threadIdx.x & 63, st = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t sid = c * LQ_STREAMS + st;
    const uint32_t* bb = blk_bits + sid * nblk;
    uint32_t* bo = blk_off + sid * nblk;
    uint64_t carry = 0;
    for (int64_t r0 = 0; r0 < nblk; r0 += 64 * kScanRounds) {
        uint32_t v[kScanRounds];
#pragma unroll
        for (int k = 0; k < kScanRounds; k++) {
            const int64_t b = r0 + 64 * k + lane;
            v[k] = b < nblk ? bb[b] : 0u;
        }
#pragma unroll
        for (int k = 0; k < kScanRounds; k++) {
            const uint32_t x = wave_incl_scan(v[k]);   // counts < 2^13, sums < 2^19
            const int64_t b = r0 + 64 * k + lane;
            if (b < nblk) bo[b] = (uint32_t)(carry + x - v[k]);
            carry += (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
        }
    }
    if (lane == 0) {
        const bool present = tables[sid].n_sym > 0;
        s_present[st] = present ? 1 : 0;
        s_nbits[st] = present ? (int64_t)carry : 0;
        stream_nbits[sid] = present ? (int64_t)carry : 0;
        stream_state[sid] = present ? (int32_t)blk_state[sid * nblk] : 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t w = 0;
        for (int k = 0; k < LQ_STREAMS; k++) {
            stream_woff[c * LQ_STREAMS + k] = w;
            if (s_present[k]) w += (s_nbits[k] + 31) / 32 + 1;
        }
        chunk_words[c] = w;
    }
}

// Tiled scan of long streams.  Tile t of stream sid covers blocks
// t * kScanTile .. + kScanTile - 1; thread i of its workgroup owns the 16
// consecutive blocks from t * kScanTile + 16 i.
__device__ __forceinline__ uint64_t block_exclusive_scan256(uint64_t v, uint64_t* part, uint64_t* total) {
    const int tid = threadIdx.x;
    part[tid] = v;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {   // inclusive Hillis-Steele scan
        const uint64_t u = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += u;
        __syncthreads();
    }
    *total = part[255];
    return tid ? part[tid - 1] : 0;
}

__global__ __launch_bounds__(256) void k_scan_tiles(const uint32_t* __restrict__ blk_bits, int64_t nblk, int64_t tiles,
                                                    uint64_t* __restrict__ tile_sum) {
    __shared__ uint64_t part[256];
    const int64_t sid = blockIdx.x / tiles, t = blockIdx.x % tiles;
    const uint32_t* bb = blk_bits + sid * nblk;
    const int64_t b0 = t * kScanTile + 16 * (int64_t)threadIdx.x;
    uint64_t s = 0;
#pragma unroll
    for (int k = 0; k < 16; k++)
        if (b0 + k < nblk) s += bb[b0 + k];
    uint64_t tot;
    block_exclusive_scan256(s, part, &tot);
    if (threadIdx.x == 0) tile_sum[sid * tiles + t] = tot;
}

// per stream: exclusive prefix of its tile sums (in place), n_bits, final state
__global__ __launch_bounds__(256) void k_scan_top(uint64_t* __restrict__ tile_sum, int64_t tiles,
                                                  const uint16_t* __restrict__ blk_state, int64_t nblk,
                                                  const lq_table* __restrict__ tables, int64_t* __restrict__ stream_nbits,
                                                  int32_t* __restrict__ stream_state) {
    __shared__ uint64_t part[256];
    const int64_t sid = blockIdx.x;
    uint64_t* ts = tile_sum + sid * tiles;
    uint64_t carry = 0;
    for (int64_t t0 = 0; t0 < tiles; t0 += 256) {   // uniform trip count
        const int64_t t = t0 + threadIdx.x;
        const uint64_t v = t < tiles ? ts[t] : 0;
        uint64_t tot;
        const uint64_t ex = block_exclusive_scan256(v, part, &tot);
        if (t < tiles) ts[t] = carry + ex;
        carry += tot;
        __syncthreads();   // part is reused by the next round
    }
    if (threadIdx.x == 0) {
        const bool present = tables[sid].n_sym > 0;
        stream_nbits[sid] = present ? (int64_t)carry : 0;
        stream_state[sid] = present ? (int32_t)blk_state[sid * nblk] : 0;
    }
}

__global__ __launch_bounds__(256) void k_scan_apply(const uint32_t* __restrict__ blk_bits, int64_t nblk, int64_t tiles,
                                                    const uint64_t* __restrict__ tile_off, uint32_t* __restrict__ blk_off) {
    __shared__ uint64_t part[256];
    const int64_t sid = blockIdx.x / tiles, t = blockIdx.x % tiles;
    const uint32_t* bb = blk_bits + sid * nblk;
    uint32_t* bo = blk_off + sid * nblk;
    const int64_t b0 = t * kScanTile + 16 * (int64_t)threadIdx.x;
    uint32_t v[16];
    uint64_t s = 0;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        v[k] = b0 + k < nblk ? bb[b0 + k] : 0u;
        s += v[k];
    }
    uint64_t tot;
    uint64_t run = tile_off[sid * tiles + t] + block_exclusive_scan256(s, part, &tot);
#pragma unroll
    for (int k = 0; k < 16; k++) {
        if (b0 + k < nblk) bo[b0 + k] = (uint32_t)run;
        run += v[k];
    }
}

// per chunk: word offset of each present stream (n_words + 1 words each) and chunk total
__global__ void k_chunk_offsets(const int64_t* __restrict__ stream_nbits, const lq_table* __restrict__ tables,
                                int64_t n_chunks, int64_t* __restrict__ stream_woff, int64_t* __restrict__ chunk_words) {
    int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n_chunks) return;
    int64_t w = 0;
    for (int st = 0; st < LQ_STREAMS; st++) {
        int64_t sid = c * LQ_STREAMS + st;
        stream_woff[sid] = w;
        if (tables[sid].n_sym > 0) w += (stream_nbits[sid] + 31) / 32 + 1;
    }
    chunk_words[c] = w;
}

// One wave per (stream, group of 32 blocks).  The group owns the stream
// words whose first bit lies in its blocks' bit range; lane l assembles words
// W0 + l + 64 k, kPackU per round with all their scratch loads in flight
// (256-byte coalesced stores).  A word's first bits come from the
// right-aligned scratch of the block holding its first bit (one funnel
// shift), the rest, when the word runs past that block's end, from the first
// bits of the next block (loaded only in those lanes, merged with a select);
// the rare word that also runs past that block, or is the stream's last and
// partly past its end, is assembled block by block.  Scratch and output words
// are addressed with 32-bit byte offsets from wave-uniform bases.  The block of
// each word comes from the blocks' first owned words fw_i = ceil(off_i / 32),
// held one per lane: within a 64-word slice, the block of word w is the last
// block with fw_i <= w, i.e. the last block starting at or before the slice
// (a ballot count) unless one of the few blocks starting inside the slice
// (another ballot, walked on the scalar unit) has fw_i <= w.  The wave of a
// stream's last group also writes the zero word after the stream.  Stream bit
// positions are 32-bit (blk_off is uint32).
constexpr int kPackBlocks = 32;
constexpr int kPackU = 4;   // words per lane per round, their scratch loads all in flight

__global__ __launch_bounds__(256) void k_chunk_pack(int64_t n_streams_total, int64_t nblk, const uint32_t* __restrict__ scratch,
                                                    const uint32_t* __restrict__ blk_off,
                                                    const int64_t* __restrict__ stream_nbits,
                                                    const int64_t* __restrict__ stream_woff,
                                                    const int64_t* __restrict__ chunk_base,
                                                    const lq_table* __restrict__ tables, uint32_t* __restrict__ words) {
    __shared__ uint32_t offs[4][kPackBlocks + 2];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int64_t gps = (nblk + kPackBlocks - 1) / kPackBlocks;   // groups per stream
    const int64_t job = (int64_t)blockIdx.x * 4 + wave;
    const int64_t sid = job / gps;
    const int64_t g0 = (job % gps) * kPackBlocks;
    if (sid >= n_streams_total || tables[sid].n_sym == 0) return;   // wave-uniform; no barrier follows
    const uint32_t nbits = (uint32_t)stream_nbits[sid];
    const int nb = (int)(nblk - g0 < kPackBlocks ? nblk - g0 : kPackBlocks);
    const uint32_t* bo = blk_off + sid * nblk;
    // offset of block g0 + i (the stream end past the last block); staged for i <= nb + 1
    auto off_glb = [&](int i) -> uint32_t { return g0 + i < nblk ? bo[g0 + i] : nbits; };
    uint32_t* of = offs[wave];
    const uint32_t myof = lane <= nb + 1 ? off_glb(lane) : 0u;
    if (lane <= nb + 1) of[lane] = myof;
    __builtin_amdgcn_wave_barrier();
    auto off_at = [&](int i) -> uint32_t { return i <= nb + 1 ? of[i] : off_glb(i); };
    // first owned word of block `lane` (blocks 0 .. nb - 1), else past every word
    const uint32_t myfw = lane < nb ? (myof + 31u) >> 5 : 0xffffffffu;
    const uint32_t W0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)((myof + 31u) >> 5));
    const uint32_t W1 = (uint32_t)__builtin_amdgcn_readlane((int)((myof + 31u) >> 5), nb);
    uint32_t* out = words + chunk_base[sid / LQ_STREAMS] + stream_woff[sid];
    // the stream's trailing zero word, from the wave of its last group
    if (g0 + nb >= nblk && lane == 0) out[((uint64_t)nbits + 31u) >> 5] = 0u;
    const uint32_t* scr0 = scratch + (sid * nblk + g0) * (int64_t)kCapW;
    constexpr uint32_t kCapBits = (uint32_t)kCapW * 32u;
    // scratch word i of the group (i < (nb + 1) * kCapW), as a 32-bit byte
    // offset from the wave-uniform base; likewise the stream's output words
    auto scr = [&](uint32_t i) -> uint32_t {
        return *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(scr0) + (i << 2));
    };
    for (uint32_t wr = W0; wr < W1; wr += 64u * kPackU) {
        uint32_t lo[kPackU], hi[kPackU], clo[kPackU], chi[kPackU];
        int blk[kPackU], take[kPackU], s2[kPackU], cs[kPackU];
        uint32_t pe[kPackU];
        bool nxt[kPackU], rare[kPackU];
#pragma unroll
        for (int u = 0; u < kPackU; u++) {
            const uint32_t ws = wr + 64u * u;   // first word of the slice (wave-uniform)
            const uint32_t w = ws + lane;
            const bool ok = w < W1;
            // blocks starting at or before the slice, and inside it
            const uint64_t at = __ballot(myfw <= ws);
            uint64_t in = __ballot(myfw > ws && myfw <= ws + 63u);
            int b = __builtin_popcountll(at) - 1;
            while (in) {
                const int i = __builtin_ctzll(in);
                in &= in - 1;
                const uint32_t fwi = (uint32_t)__builtin_amdgcn_readlane((int)myfw, i);
                b = w >= fwi ? i : b;
            }
            const uint32_t p = 32u * (ok ? w : W0);
            if (!ok) b = 0;
            const uint32_t ob = of[b], oe = of[b + 1], on = of[b + 2];
            const uint32_t end = p + 32u < nbits ? p + 32u : nbits;
            const uint32_t e1 = end < oe ? end : oe;
            const uint32_t sp = kCapBits - (oe - ob) + (p - ob);   // scratch bit of p
            const uint32_t k0 = sp >> 5;
            const uint32_t i0 = (uint32_t)b * (uint32_t)kCapW + k0;
            lo[u] = scr(i0);
            hi[u] = scr(k0 + 1 < (uint32_t)kCapW ? i0 + 1 : i0);
            // a word running past its block's end continues with the first bits
            // of block b + 1 (when that block is not empty): load them in the
            // lanes that need them; they are consumed unconditionally below, so
            // no load is left pending into the next round
            const uint32_t sp1 = kCapBits - (on - oe);            // scratch bit of block b + 1's first bit
            const uint32_t k1 = sp1 >> 5;
            const bool cont = ok && e1 < end;
            nxt[u] = cont && on > oe;
            clo[u] = 0u;
            chi[u] = 0u;
            if (nxt[u]) {
                const uint32_t i1 = (uint32_t)(b + 1) * (uint32_t)kCapW + k1;
                clo[u] = scr(i1);
                chi[u] = scr(k1 + 1 < (uint32_t)kCapW ? i1 + 1 : i1);
            }
            const uint32_t e2 = end < on ? end : on;
            // rare: block b + 1 is empty, ends inside the word too, or the word
            // is the stream's last and partly past its end (its unused bits
            // must be zero); otherwise the two segments fill all 32 bits
            rare[u] = cont && e2 != p + 32u;
            blk[u] = b;
            take[u] = (int)(e1 - p);   // 1 .. 32
            s2[u] = (int)(sp & 31u);
            cs[u] = (int)(sp1 & 31u);
            pe[u] = e1;
        }
#pragma unroll
        for (int u = 0; u < kPackU; u++) {
            const uint32_t w = wr + 64u * u + lane;
            const int got = take[u];
            uint32_t res = __builtin_amdgcn_alignbit(hi[u], lo[u], (uint32_t)s2[u]) & (0xffffffffu >> ((32 - got) & 31));
            // the next block's first bits fill the rest of the word (got < 32 there)
            const uint32_t seg2 = __builtin_amdgcn_alignbit(chi[u], clo[u], (uint32_t)cs[u]) << (got & 31);
            res |= nxt[u] ? seg2 : 0u;
            if (rare[u]) {
                // block by block from block b + 1: empty blocks are skipped,
                // a block ending inside the word gives only its bits
                res &= 0xffffffffu >> ((32 - got) & 31);
                const uint32_t end = 32u * w + 32u < nbits ? 32u * w + 32u : nbits;
                uint32_t p = pe[u];
                int gb = got;
                int b = blk[u] + 1;
                while (p < end) {
                    const uint32_t ob = off_at(b), oe = off_at(b + 1);
                    if (oe > ob) {
                        const uint32_t e1 = end < oe ? end : oe;
                        const int tk2 = (int)(e1 - p);
                        const uint32_t sp = kCapBits - (oe - ob) + (p - ob);
                        const uint32_t* sc = scr0 + (int64_t)b * kCapW;
                        uint64_t y = sc[sp >> 5];
                        if ((int)(sp & 31u) + tk2 > 32) y |= (uint64_t)sc[(sp >> 5) + 1] << 32;
                        y >>= (sp & 31u);
                        res |= (tk2 == 32 ? (uint32_t)y : (uint32_t)y & ((1u << tk2) - 1u)) << gb;
                        gb += tk2;
                        p = e1;
                    }
                    b++;
                }
            }
            if (w < W1) *reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(out) + (w << 2)) = res;
        }
    }
}

// ------------------------------------------------------------ chunk decode --

// Decoder LUT of every chunk stream (lut_entry format, lq_decode.h).
// mode 0 (decode attention): stream st of a chunk sits at row st & 7 (the 8
// LUTs of one coset form one LDS block) and the symbol field is the alphabet
// index.  mode 1 (chunk decoder): row st & 15 (the 16 LUTs of a chunk form
// one LDS block), and the symbol field is biased (chunk_biased) when the
// chunk's alphabets allow it.
__global__ __launch_bounds__(256) void k_chunk_lut(const lq_table* __restrict__ tables, uint32_t* __restrict__ lut,
                                                   int mode) {
    __shared__ int32_t fr[LQ_MAXSYM];
    __shared__ int32_t cum[LQ_MAXSYM + 1];
    const int64_t sid = blockIdx.x;
    const lq_table* T = tables + sid;
    const int n = T->n_sym;
    if (n == 0) return;
    for (int i = threadIdx.x; i < n; i += 256) fr[i] = (int32_t)enc_f(T->enc[i]);
    __syncthreads();
    exclusive_scan_array<BlockGroup>(fr, n, cum);
    const int st = (int)(sid % LQ_STREAMS);
    const uint32_t row = (uint32_t)st & (mode ? 15u : 7u);
    uint32_t bias = 0;
    if (mode && chunk_biased(tables + (sid - st))) bias = (uint32_t)(T->lo + ((st & 7) < 7 ? 512 : 256));
    for (int slot = threadIdx.x; slot < kL; slot += 256) {
        int lo = 0, hi = n - 1;   // largest s with cum[s] <= slot
        while (lo < hi) {
            int mid = (lo + hi + 1) >> 1;
            if (cum[mid] <= slot) lo = mid; else hi = mid - 1;
        }
        lut[sid * kL + slot] = lut_entry((uint32_t)lo + bias, (uint32_t)(fr[lo] + slot - cum[lo]), row);
    }
}

// Whole-line chunk decoder.
//
// Workgroup: 64 consecutive blocks of one chunk, 16 lanes per block (one
// wave holds 4 blocks): lane (block b, coset c, coordinate idx) decodes stream
// c * 8 + idx of block b with LineLane, in phases of 8 steps.  Step j of a
// phase stages the symbol index of coset-c vector `st + j` of the block at
// rank slot (st + j) % 16 of the (block, coset) staging, so no lane walks the
// coset bitmap per symbol.  After each phase the block's 16 lanes flush the
// output in whole 128-byte lines (8 vectors): a line is flushed once both
// cosets have staged every vector in it; a flushed vector's rank in its coset
// is the flushed count plus a popcount of the coset-1 bitmap below it.  A
// phase flushes at most two lines (16 consecutive vectors, 256 bytes, one
// per lane of the block's row): a second round for lines 3 and 4 left most
// of its lanes idle and cost more than the extra phases the cap adds (the
// first flushable line is always taken, so the cap never stalls the loop).
// A coset runs a phase only if the 8 vectors it stages fit the ring next to
// its unflushed ones (st - flushed <= 8).  That never blocks for good: the
// first unflushed line holds at most 8 vectors of each coset, so a coset
// that has not staged all of them has fewer than 8 unflushed and may run.
// HEADS_ALIGNED: bph is a multiple of the block size, so a block lies in one
// head.  DITHER: the chunk's dither (dither8, seed dseed[chunk]) is
// subtracted from each lattice point before scaling.
constexpr int kDecBlocks = 64;                  // blocks per decode workgroup
constexpr int kDecThreads = 16 * kDecBlocks;    // 1024
constexpr int kDecStage = 16;                   // staged vectors per (block, coset)
// Staging of (block b, coset c): group b * 2 + c, 16 slots of 8 u16, padded to
// 68 words so that group bases fall on banks 4 g (mod 64): the 8 groups of a
// wave write their slots j or j + 8 on disjoint banks.
constexpr int kDecGroupU16 = 136;

__device__ __forceinline__ int dpp_ror8(int v) {   // lane l <- lane l ^ 8 within each 16-lane row
    return __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false);
}

template <int OUT_DT, bool HEADS_ALIGNED, bool DITHER, bool ROT = false, bool ESC = false>
__global__ __launch_bounds__(kDecThreads) void k_chunk_decode(
        const uint32_t* __restrict__ words, const int64_t* __restrict__ chunk_base, const int64_t* __restrict__ stream_woff,
        const uint32_t* __restrict__ blk_off, const int64_t* __restrict__ stream_nbits,
        const uint16_t* __restrict__ blk_state, const uint8_t* __restrict__ coset_bits,
        const lq_table* __restrict__ tables, const uint16_t* __restrict__ scale16, const uint32_t* __restrict__ lutg,
        int64_t n_chunks, int64_t n_heads, int64_t bph, int64_t nblk, int64_t gpw, void* __restrict__ out,
        const int64_t* __restrict__ dseed, const float* __restrict__ signs, int lpr, float rdiv,
        const int32_t* __restrict__ esc_k, const int64_t* __restrict__ fine_off, const uint32_t* __restrict__ fine) {
    __shared__ uint32_t lut[LQ_STREAMS * kL];                               // 64 KB
    __shared__ uint32_t ring[kDecThreads / 64][kLineRing][64];              // 48 KB
    __shared__ __align__(16) uint16_t stg[kDecBlocks * 2 * kDecGroupU16];   // 34 KB
    __shared__ uint32_t bm1[kDecBlocks][kBlk / 32 + 1];                     // coset-1 bits, one zero word after each row
    const int tid = threadIdx.x;
    const float rrcp = ROT ? 1.0f / rdiv : 1.0f;   // the rotation's RN(1 / sqrt(head_dim))
    const int64_t V = n_heads * bph;
    const int64_t groups = (nblk + kDecBlocks - 1) / kDecBlocks;   // per chunk
    const int64_t total = n_chunks * groups;
    const int64_t first = (int64_t)blockIdx.x * gpw;
    const int64_t last = first + gpw < total ? first + gpw : total;
    const int wave = tid >> 6, lane = tid & 63;
    int64_t lut_chunk = -1;
    // The workgroup walks groups first .. last - 1 (64 blocks each); its LUTs
    // are reloaded, between two barriers, only when the chunk changes.  Each
    // wave stages its own 4 blocks' bitmaps and moves to its next blocks
    // without waiting for the other waves.
    for (int64_t gi = first; gi < last; gi++) {
    const int64_t chunk = gi / groups;
    const int64_t gbase = (gi % groups) * kDecBlocks;
    if (chunk != lut_chunk) {
        __syncthreads();   // every wave is done with the previous chunk's LUTs
        const uint4* src = reinterpret_cast<const uint4*>(lutg + chunk * LQ_STREAMS * kL);
        uint4* dst = reinterpret_cast<uint4*>(lut);
        for (int i = tid; i < LQ_STREAMS * kL / 4; i += kDecThreads) dst[i] = src[i];
        __syncthreads();
        lut_chunk = chunk;
    }
    __builtin_amdgcn_wave_barrier();
    for (int i = lane; i < 4 * (kBlk / 32 + 1); i += 64) {
        const int bl = wave * 4 + i / (kBlk / 32 + 1), w = i % (kBlk / 32 + 1);
        const int64_t g = gbase + bl;
        uint32_t m = 0;
        if (w < kBlk / 32 && g < nblk) {
            m = reinterpret_cast<const uint32_t*>(coset_bits + (chunk * nblk + g) * (kBlk / 8))[w];
            const int64_t lim = V - g * kBlk - 32 * w;
            m = lim >= 32 ? m : (lim <= 0 ? 0u : m & ((1u << lim) - 1u));
        }
        bm1[bl][w] = m;
    }
    __builtin_amdgcn_wave_barrier();
    {
    const int b = tid >> 4, c = (tid >> 3) & 1, idx = tid & 7, l16 = tid & 15;
    const int64_t g = gbase + b;
    if (g >= nblk) continue;   // whole blocks (16-lane rows) skip together
    const int64_t vfirst = g * kBlk;                 // first vector of the block, within the chunk
    const int valid = (int)(V - vfirst < kBlk ? V - vfirst : kBlk);
    // coset-1 count of the block from its bitmap (equal to blk_n1 for every
    // chunk the encoder wrote); counting it here ties the loop below to the
    // bitmap, so it ends even if the metadata disagrees with it
    int n1 = 0;
#pragma unroll
    for (int w = 0; w < kBlk / 32; w++) n1 += __builtin_popcount(bm1[b][w]);
    const int n = c ? n1 : valid - n1;
    const lq_table* T = tables + chunk * LQ_STREAMS;
    // escaped chunk (coarse symbols plus raw low bits, alphabets beyond L):
    // the generic path with the low bits merged in
    const int32_t* const ekc = ESC && esc_k ? esc_k + chunk * 8 : nullptr;
    bool esc = false;
    EscCoords ec;
    if (ESC && ekc) {
        ec.init(ekc, fine_off + chunk * 8, fine);
#pragma unroll
        for (int j = 0; j < 8; j++) esc = esc || ec.k[j] != 0;
    }
    const bool lut_biased = chunk_biased(T);   // the LUT's symbol fields (k_chunk_lut decides the same way)
    const bool biased = !esc && lut_biased;
    CosetConsts cc0, cc1;   // per-coset alphabet lows, for chunks whose fields are not biased
    if (!biased) {
        cc0.init(T, 0);
        cc1.init(T + 8, 1);
    }
    float sc;
    half2_t sc2;
    const float* sgp = nullptr;   // ROT: the head's sign row
    auto set_scale = [&](int64_t head) {
        const uint16_t s16 = scale16[chunk * n_heads + head];
        sc = h2f(s16);
        const _Float16 sh = __builtin_bit_cast(_Float16, s16);
        sc2 = half2_t{sh, sh};
        if (ROT) sgp = signs + (chunk * n_heads + head) * (8 * (int64_t)lpr);
    };
    const int64_t head0 = vfirst / bph;
    set_scale(head0);
    int64_t head_end = (head0 + 1) * bph;            // first chunk vector of the next head

    const int st_id = c * 8 + idx;
    const int64_t sid = chunk * LQ_STREAMS + st_id;
    LineLane d;
    if (n > 0) {
        const int64_t task = sid * nblk + g;
        const int64_t end_bit = g + 1 < nblk ? (int64_t)blk_off[task + 1] : stream_nbits[sid];
        d.init(words + chunk_base[chunk] + stream_woff[sid], blk_off[task], end_bit, blk_state[task], lut, st_id,
               &ring[tid >> 6][0][tid & 63]);
    } else {
        d.inflight = false;
    }
    const char* const lutb = reinterpret_cast<const char*>(lut);
    using OutT = typename std::conditional<OUT_DT == LQ_F32, float, uint16_t>::type;
    OutT* const ob = reinterpret_cast<OutT*>(out) + (chunk * V + vfirst) * 8;
    const uint64_t dkey = DITHER ? mix64((uint64_t)dseed[chunk]) : 0u;
    const uint32_t* const bmr = bm1[b];
    uint16_t* const my_stg = &stg[(b * 2 + c) * kDecGroupU16 + idx];
    const int u = (l16 & 1) + 1;     // lines of the flush candidate this lane checks

    float pend[ROT ? 8 : 1];         // ROT: butterfly stages of a deferred first half-row (lanes 0..7)
    int st = 0;                      // vectors of my coset staged (symbols of my stream decoded)
    int fpos = 0, fr0 = 0, fr1 = 0;  // flushed block positions and flushed ranks per coset (block-uniform)
    while (fpos < valid) {
        __builtin_amdgcn_wave_barrier();
        const bool more = st < n;
        d.boundary(more);
        if (more && st - (c ? fr1 : fr0) <= kDecStage - 8) {
            // st % 8 == 0 here, so the phase's slots do not wrap; a last phase
            // with fewer than 8 symbols stages garbage in slots of ranks >= n,
            // which hold no unflushed rank (st + 8 - flushed <= 16) and are never read
            d.phase(my_stg + (st & (kDecStage - 1)) * 8, lutb);
            st = n - st < kPhase ? n : st + kPhase;
        }
        __builtin_amdgcn_wave_barrier();
        const int st_o = dpp_ror8(st);
        const int s0 = c ? st_o : st, s1 = c ? st : st_o;
        // coset-1 bits of positions fpos .. fpos + 31; lanes 0 and 1 of the
        // block's row check whether the first 1 and 2 lines can be flushed (the
        // answers are monotone, so their count is the number of lines flushed)
        const int wi = fpos >> 5;
        const uint32_t W = __builtin_amdgcn_alignbit(bmr[wi + 1], bmr[wi], (uint32_t)(fpos & 31));
        const int rest = valid - fpos;
        const int np = rest < 8 * u ? rest : 8 * u;                  // 1 <= np <= 16
        const int p1 = __builtin_popcount(W << ((32 - np) & 31));   // coset-1 vectors among them
        const bool ok = 8 * (u - 1) < rest && fr0 + np - p1 <= s0 && fr1 + p1 <= s1;
        const uint64_t bal = __builtin_amdgcn_ballot_w64(ok);
        int nl = __builtin_popcountll((bal >> (tid & 48)) & 0x3ull);   // 0, 1 or 2 lines
        // ROT: a flush that starts in the middle of a 16-vector row takes one
        // line, the row's second half, so the next flushes start on a row
        // again (a 16-vector flush from the middle of a row runs the
        // butterflies of two rows for one row's stores)
        if (ROT && (fpos & 8) && nl > 1) nl = 1;
        const int F = 8 * nl < rest ? 8 * nl : rest;   // positions flushed this phase (<= 16)
        // fp32 output row of position p (fpos <= p < fpos + F): the lattice
        // point from its staged symbols, dither removed, times the head's scale
        auto lattice_y = [&](int p, float y[8]) {
            const int q = p - fpos;
            const bool cp = (W >> q) & 1u;
            const int n1b = __builtin_popcount(W & ((1u << q) - 1u));
            const int rank = cp ? fr1 + n1b : fr0 + q - n1b;
            const uint4 r = *reinterpret_cast<const uint4*>(&stg[(b * 2 + cp) * kDecGroupU16 + (rank & (kDecStage - 1)) * 8]);
            if (!HEADS_ALIGNED && vfirst + p >= head_end) {
                const int64_t head = (vfirst + p) / bph;
                head_end = (head + 1) * bph;
                set_scale(head);
            }
            if (biased) {
                lattice_biased_f32(r, cp ? 0.5f : 0.f, y);
            } else if (ESC && esc) {
                CosetConsts cs;
                cs.pick(cp, cc0, cc1);
                lattice_escaped_f32(r, cs, lut_biased, ec, vfirst + p, y);
            } else {
                CosetConsts cs;
                cs.pick(cp, cc0, cc1);
                cs.deq_f32(r, 1.0f, y);   // the lattice point itself (exact)
            }
            if constexpr (DITHER) {
                float dd[8];
                dither8(dkey, vfirst + p, dd);
#pragma unroll
                for (int j = 0; j < 8; j++) y[j] = (y[j] - dd[j]) * sc;
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) y[j] *= sc;
            }
        };
        if constexpr (ROT) {
            // Lane l16 stores the positions p == l16 (mod 16) of the flush, so a
            // 16-vector row's first half always sits in lanes 0..7 and its second
            // half in lanes 8..15.  Rows of lpr <= 8 vectors lie inside one line
            // and are rotated back whole.  When a 16-vector row's first line
            // flushes before its second, that half's butterfly stages (h <= 32)
            // wait in registers (pend) and its store is deferred; when the second
            // line comes both halves take the last stage (h = 64) together: the
            // operations and their order are those of the whole-row transform.
            for (int base = fpos & ~15; F > 0 && base < fpos + F; base += 16) {
                const int p = base + l16;
                const bool mine = p >= fpos && p < fpos + F;
                float y[8];
                if (mine) lattice_y(p, y);
                float sg[8];
                load_signs8(sgp + 8 * (l16 & (lpr - 1)), sg);
                if (lpr < 16) {
                    if (mine) {
                        rht_lanes(y, sg, l16 & (lpr - 1), lpr, rdiv, rrcp, true);
                        store8(ob, OUT_DT, p, y);
                    }
                } else {
                    const bool fh = base >= fpos && base + 8 <= fpos + F;   // the row's first line flushes now
                    const bool sh = base + 16 <= fpos + F;                   // its second line flushes now
                    if (mine) fwht_stages(y, l16 & 7, 8);
                    if (!sh) {
                        if (fh && mine) {
#pragma unroll
                            for (int j = 0; j < 8; j++) pend[j] = y[j];
                        }
                    } else {
                        if (!fh && l16 < 8) {
#pragma unroll
                            for (int j = 0; j < 8; j++) y[j] = pend[j];
                        }
                        fwht_cross(y, l16, 8);
                        div_sqrt_dim8(y, rdiv, rrcp);
#pragma unroll
                        for (int j = 0; j < 8; j++) y[j] = y[j] * sg[j];
                        store8(ob, OUT_DT, base + l16, y);
                    }
                }
            }
        } else {
            for (int r0 = 0; r0 < F; r0 += 16) {
                const int q = r0 + l16;
                if (q < F) {
                    const int p = fpos + q;
                    if (!DITHER && OUT_DT == LQ_F16 && biased) {
                        const bool cp = (W >> q) & 1u;
                        const int n1b = __builtin_popcount(W & ((1u << q) - 1u));
                        const int rank = cp ? fr1 + n1b : fr0 + q - n1b;
                        const uint4 r = *reinterpret_cast<const uint4*>(
                            &stg[(b * 2 + cp) * kDecGroupU16 + (rank & (kDecStage - 1)) * 8]);
                        if (!HEADS_ALIGNED && vfirst + p >= head_end) {
                            const int64_t head = (vfirst + p) / bph;
                            head_end = (head + 1) * bph;
                            set_scale(head);
                        }
                        const _Float16 o = cp ? (_Float16)0.5f : (_Float16)0.0f;
                        reinterpret_cast<uint4*>(ob)[p] = deq_biased_f16(r, half2_t{o, o}, sc2);
                    } else {
                        float y[8];
                        lattice_y(p, y);
                        store8(ob, OUT_DT, p, y);
                    }
                }
            }
        }
        const int f1 = __builtin_popcount(W) - __builtin_popcount((uint32_t)((uint64_t)W >> F));   // 0 <= F <= 16
        fr1 += f1;
        fr0 += F - f1;
        fpos += F;
    }
    }
    }
}

// ------------------------------------------------------- generic tables --

__global__ __launch_bounds__(256) void k_build_tables(const int64_t* __restrict__ counts, const int64_t* __restrict__ count_off,
                                                      const int32_t* __restrict__ n_sym, int32_t* __restrict__ freqs_out,
                                                      int32_t* __restrict__ cum_out, int32_t* __restrict__ lookup,
                                                      int32_t* __restrict__ status) {
    __shared__ int64_t cnt[kL];
    __shared__ int32_t fr[kL];
    __shared__ NpScratch ns;
    __shared__ int16_t perm[kL];
    __shared__ int s_st;
    const int t = blockIdx.x;
    const int n = n_sym[t];
    const int64_t o = count_off[t];
    if (n <= 0 || n > kL) {
        if (threadIdx.x == 0) status[t] = LQ_ST_ALPHABET;
        return;
    }
    for (int i = threadIdx.x; i < n; i += 256) cnt[i] = counts[o + i];
    if (threadIdx.x == 0) s_st = 0;
    __syncthreads();
    __shared__ int64_t kk[kL];
    __shared__ int8_t inset[kL];
    normalise<BlockGroup>(cnt, n, fr, perm, kk, inset, &ns);
    __shared__ int32_t cum[kL + 1];
    exclusive_scan_array<BlockGroup>(fr, n, cum);
    for (int i = threadIdx.x; i < n; i += 256) freqs_out[o + i] = fr[i];
    for (int i = threadIdx.x; i <= n; i += 256) cum_out[o + t + i] = cum[i];
    for (int slot = threadIdx.x; slot < kL; slot += 256) {   // largest s with cum[s] <= slot
        int lo = 0, hi = n - 1;
        while (lo < hi) {
            int mid = (lo + hi + 1) >> 1;
            if (cum[mid] <= slot) lo = mid; else hi = mid - 1;
        }
        lookup[(int64_t)t * kL + slot] = lo;
    }
    if (threadIdx.x == 0) status[t] = s_st;
}

// ------------------------------------------------------ generic streams --

// Serial encode of one stream per lane, then the bits are laid out in the
// reference's word order (n_words + 1 words, last zero).
__global__ void k_encode_streams(const int32_t* __restrict__ idx, const int64_t* __restrict__ sym_off,
                                 const int64_t* __restrict__ nsym, const int32_t* __restrict__ freqs,
                                 const int32_t* __restrict__ cum, const int64_t* __restrict__ tab_off, int32_t n_streams,
                                 uint32_t* __restrict__ scratch, uint32_t* __restrict__ words,
                                 const int64_t* __restrict__ word_off, int64_t* __restrict__ state_out,
                                 int64_t* __restrict__ nbits_out) {
    int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_streams) return;
    const int64_t n = nsym[t];
    const int32_t* id = idx + sym_off[t];
    const int32_t* F = freqs + tab_off[t];
    const int32_t* C = cum + tab_off[t];
    const int64_t cap = (10 * n + 31) / 32 + 2;
    uint32_t* scr = scratch + word_off[t];
    uint32_t* out = words + word_off[t];
    int64_t wpos = cap - 1;
    uint64_t acc = 0;
    uint32_t nacc = 0;
    int64_t total = 0;
    uint32_t x = kL;
    for (int64_t j = n - 1; j >= 0; j--) {
        uint32_t f = (uint32_t)F[id[j]], cf = (uint32_t)C[id[j]];
        uint32_t e = enc_pack(f, cf);
        uint32_t k, xin = x;
        x = enc_step(x, e, &k);
        uint64_t r = ((uint64_t)__builtin_bitreverse32(xin) << k) >> 32;
        acc = (acc << k) | r;
        nacc += k;
        total += k;
        if (nacc >= 32) { nacc -= 32; scr[wpos--] = (uint32_t)(acc >> nacc); }
    }
    if (nacc) scr[wpos] = (uint32_t)(acc << (32 - nacc));
    const int64_t nw = (total + 31) / 32;
    const int64_t base = cap * 32 - total;   // scratch bit position of stream bit 0
    for (int64_t w = 0; w < nw; w++) {
        int64_t sp = base + 32 * w;
        int64_t wi = sp >> 5;
        int sh = (int)(sp & 31);
        int take = (int)(total - 32 * w < 32 ? total - 32 * w : 32);
        uint64_t v = scr[wi];
        if (sh + take > 32) v |= (uint64_t)scr[wi + 1] << 32;
        v >>= sh;
        out[w] = take == 32 ? (uint32_t)v : (uint32_t)v & ((1u << take) - 1u);
    }
    out[nw] = 0u;
    state_out[t] = x;
    nbits_out[t] = total;
}

// _rans_decode_kernel semantics (core/gpu_ans.py:175-235): one stream per lane,
// renormalisation reads min(needed, n_bits - bit_pos) bits.
__global__ void k_decode_streams(const int32_t* __restrict__ bits, const int32_t* __restrict__ bit_off,
                                 const int32_t* __restrict__ nbits, const int32_t* __restrict__ init,
                                 const int32_t* __restrict__ ndec, const int32_t* __restrict__ lookup,
                                 const int32_t* __restrict__ freqs, const int32_t* __restrict__ cum,
                                 const int32_t* __restrict__ alphabet, const int32_t* __restrict__ tid_,
                                 int32_t max_sym, const int32_t* __restrict__ out_off, int32_t n_streams,
                                 int64_t* __restrict__ out) {
    int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_streams) return;
    const uint32_t* wb = reinterpret_cast<const uint32_t*>(bits);
    const int64_t boff = bit_off[t];
    const int64_t nb = nbits[t];
    const int n = ndec[t];
    const int tb = tid_[t];
    const int32_t* LU = lookup + (int64_t)tb * kL;
    const int32_t* F = freqs + (int64_t)tb * max_sym;
    const int32_t* C = cum + (int64_t)tb * max_sym;
    const int32_t* A = alphabet + (int64_t)tb * max_sym;
    int64_t* o = out + out_off[t];
    uint32_t x = (uint32_t)init[t];
    int64_t pos = 0;
    for (int i = 0; i < n; i++) {
        uint32_t slot = x & (kL - 1);
        int si = LU[slot];
        o[i] = A[si];
        x = (uint32_t)F[si] * (x >> 10) + slot - (uint32_t)C[si];
        if (x < (uint32_t)kL) {
            int64_t k = (int64_t)__clz((int)x) - 21;
            if (k > nb - pos) k = nb - pos;
            for (int64_t q = 0; q < k; q++) {
                int64_t ab = boff + pos + q;
                x = (x << 1) | ((wb[ab >> 5] >> (ab & 31)) & 1u);
            }
            pos += k;
        }
    }
}

template <typename SymT>
int encode_launch(const SymT* d_sym, const uint32_t* d_blk_n1, int64_t n_chunks, int64_t n_vectors,
                  const lq_table* d_tables, void* d_work, uint32_t* d_blk_off, uint16_t* d_blk_state,
                  int64_t* d_stream_nbits, int32_t* d_stream_state, int64_t* d_stream_woff, int64_t* d_chunk_words,
                  hipStream_t s) {
    if (n_chunks <= 0 || n_vectors <= 0) return LQ_ERR_ARG;
    const int64_t nblk = (n_vectors + kBlk - 1) / kBlk;
    EncWork w = enc_layout(n_chunks, n_vectors);
    uint32_t* bits = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(d_work) + w.bits);
    uint32_t* scratch = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(d_work) + w.scratch);
    const int64_t groups = (nblk + kEncBlocks - 1) / kEncBlocks;
    hipLaunchKernelGGL((k_chunk_encode<SymT>), dim3((unsigned)groups, (unsigned)n_chunks), dim3(256), 0, s, d_sym,
                       d_blk_n1, nblk, n_vectors, d_tables, bits, scratch, d_blk_state);
    if (nblk > kScanTile) {
        const int64_t tiles = (nblk + kScanTile - 1) / kScanTile;
        uint64_t* tsum = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(d_work) + w.tiles);
        const dim3 tg((unsigned)(tiles * n_chunks * LQ_STREAMS));   // (stream, tile) = divmod(block, tiles)
        hipLaunchKernelGGL(k_scan_tiles, tg, dim3(256), 0, s, bits, nblk, tiles, tsum);
        hipLaunchKernelGGL(k_scan_top, dim3((unsigned)(n_chunks * LQ_STREAMS)), dim3(256), 0, s, tsum, tiles, d_blk_state,
                           nblk, d_tables, d_stream_nbits, d_stream_state);
        hipLaunchKernelGGL(k_scan_apply, tg, dim3(256), 0, s, bits, nblk, tiles, tsum, d_blk_off);
        hipLaunchKernelGGL(k_chunk_offsets, dim3((unsigned)((n_chunks + 63) / 64)), dim3(64), 0, s, d_stream_nbits,
                           d_tables, n_chunks, d_stream_woff, d_chunk_words);
    } else {
        hipLaunchKernelGGL(k_chunk_scan_offsets, dim3((unsigned)n_chunks), dim3(64 * LQ_STREAMS), 0, s, bits,
                           d_blk_state, d_tables, nblk, d_blk_off, d_stream_nbits, d_stream_state, d_stream_woff,
                           d_chunk_words);
    }
    return launch_status();
}

}  // namespace

extern "C" {

int lq_chunk_tables(const uint32_t* d_hist, int64_t n_chunks, lq_table* d_tables, int32_t* d_status, hipStream_t s) {
    if (n_chunks <= 0) return LQ_ERR_ARG;
    const int64_t ns = n_chunks * LQ_STREAMS;
    hipLaunchKernelGGL(k_chunk_tables_wave, dim3((unsigned)((ns + kTabWaves - 1) / kTabWaves)), dim3(64 * kTabWaves), 0,
                       s, d_hist, ns, d_tables, d_status);
    return launch_status();
}

int64_t lq_chunk_encode_workspace(int64_t n_chunks, int64_t n_vectors) {
    if (n_chunks <= 0 || n_vectors <= 0) return -1;
    return enc_layout(n_chunks, n_vectors).total;
}

int lq_chunk_encode(const int8_t* d_sym, const uint32_t* d_blk_n1, int64_t n_chunks, int64_t n_vectors,
                    const lq_table* d_tables, void* d_work, uint32_t* d_blk_off, uint16_t* d_blk_state,
                    int64_t* d_stream_nbits, int32_t* d_stream_state, int64_t* d_stream_woff, int64_t* d_chunk_words,
                    hipStream_t s) {
    return encode_launch(d_sym, d_blk_n1, n_chunks, n_vectors, d_tables, d_work, d_blk_off, d_blk_state, d_stream_nbits,
                         d_stream_state, d_stream_woff, d_chunk_words, s);
}

int lq_chunk_encode_wide(const int16_t* d_sym, const uint32_t* d_blk_n1, int64_t n_chunks, int64_t n_vectors,
                         const lq_table* d_tables, void* d_work, uint32_t* d_blk_off, uint16_t* d_blk_state,
                         int64_t* d_stream_nbits, int32_t* d_stream_state, int64_t* d_stream_woff, int64_t* d_chunk_words,
                         hipStream_t s) {
    return encode_launch(d_sym, d_blk_n1, n_chunks, n_vectors, d_tables, d_work, d_blk_off, d_blk_state, d_stream_nbits,
                         d_stream_state, d_stream_woff, d_chunk_words, s);
}

int lq_chunk_tables_wide(const uint32_t* d_hist, const int32_t* d_minmax, int64_t n_chunks, lq_table* d_tables,
                         int32_t* d_status, hipStream_t s) {
    if (n_chunks <= 0 || !d_hist || !d_minmax) return LQ_ERR_ARG;
    hipLaunchKernelGGL((k_chunk_tables<true>), dim3((unsigned)(n_chunks * LQ_STREAMS)), dim3(256), 0, s, d_hist, d_minmax,
                       d_tables, d_status);
    return launch_status();
}

int lq_chunk_pack(int64_t n_chunks, int64_t n_vectors, const lq_table* d_tables, const void* d_work,
                  const uint32_t* d_blk_off, const int64_t* d_stream_nbits, const int64_t* d_stream_woff,
                  const int64_t* d_chunk_base, uint32_t* d_words, hipStream_t s) {
    if (n_chunks <= 0 || n_vectors <= 0) return LQ_ERR_ARG;
    const int64_t nblk = (n_vectors + kBlk - 1) / kBlk;
    EncWork w = enc_layout(n_chunks, n_vectors);
    const uint32_t* scratch = reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(d_work) + w.scratch);
    const int64_t ns_total = n_chunks * LQ_STREAMS;
    const int64_t jobs = ns_total * ((nblk + kPackBlocks - 1) / kPackBlocks);
    hipLaunchKernelGGL(k_chunk_pack, dim3((unsigned)((jobs + 3) / 4)), dim3(256), 0, s, ns_total, nblk, scratch,
                       d_blk_off, d_stream_nbits, d_stream_woff, d_chunk_base, d_tables, d_words);
    return launch_status();
}

static int chunk_decode_launch(const uint32_t* d_words, const int64_t* d_chunk_base, const int64_t* d_stream_woff,
                               const uint32_t* d_blk_off, const int64_t* d_stream_nbits, const uint16_t* d_blk_state,
                               const uint8_t* d_coset_bits, const lq_table* d_tables, const uint16_t* d_scale16,
                               int64_t n_chunks, int64_t n_heads, int64_t bph, uint32_t* d_lut_work, void* d_out,
                               int out_dtype, const int64_t* d_dither_seed, int head_dim, const float* d_signs,
                               const int32_t* d_esc_k, const int64_t* d_fine_off, const uint32_t* d_fine,
                               hipStream_t s) {
    if (n_chunks <= 0 || n_heads <= 0 || bph <= 0 || out_dtype < 0 || out_dtype > 2) return LQ_ERR_ARG;
    if (d_esc_k && (!d_fine_off || !d_fine)) return LQ_ERR_ARG;
    const int64_t V = n_heads * bph;
    const int64_t nblk = (V + kBlk - 1) / kBlk;
    hipLaunchKernelGGL(k_chunk_lut, dim3((unsigned)(n_chunks * LQ_STREAMS)), dim3(256), 0, s, d_tables, d_lut_work, 1);
    const int64_t groups = n_chunks * ((nblk + kDecBlocks - 1) / kDecBlocks);
    const int64_t cus = device_cus();
    const int64_t gpw = (groups + cus - 1) / cus;   // groups per workgroup: one workgroup per CU
    const dim3 grid((unsigned)((groups + gpw - 1) / gpw));
    const bool aligned = bph % kBlk == 0;
    const int lpr = d_signs ? head_dim / 8 : 1;
    const float div = d_signs ? (float)sqrt((double)head_dim) : 1.0f;
    // escaped chunks get their own instantiations (the escape constants would
    // otherwise cost registers in every decoder)
#define LQ_DECODE_E(DT, AL, DI, RO, ES)                                                                           \
    hipLaunchKernelGGL((k_chunk_decode<DT, AL, DI, RO, ES>), grid, dim3(kDecThreads), 0, s, d_words, d_chunk_base,      \
                       d_stream_woff, d_blk_off, d_stream_nbits, d_blk_state, d_coset_bits, d_tables, d_scale16,       \
                       d_lut_work, n_chunks, n_heads, bph, nblk, gpw, d_out, d_dither_seed, d_signs, lpr, div,         \
                       d_esc_k, d_fine_off, d_fine)
#define LQ_DECODE(DT, AL, DI, RO)                                                                                 \
    do {                                                                                                          \
        if (d_esc_k) LQ_DECODE_E(DT, AL, DI, RO, true); else LQ_DECODE_E(DT, AL, DI, RO, false);                  \
    } while (0)
#define LQ_DECODE_DT(DT, RO)                                                                                      \
    do {                                                                                                          \
        if (d_dither_seed) { if (aligned) LQ_DECODE(DT, true, true, RO); else LQ_DECODE(DT, false, true, RO); }   \
        else { if (aligned) LQ_DECODE(DT, true, false, RO); else LQ_DECODE(DT, false, false, RO); }               \
    } while (0)
    if (d_signs) {
        if (out_dtype == LQ_F16) LQ_DECODE_DT(LQ_F16, true);
        else if (out_dtype == LQ_BF16) LQ_DECODE_DT(LQ_BF16, true);
        else LQ_DECODE_DT(LQ_F32, true);
    } else {
        if (out_dtype == LQ_F16) LQ_DECODE_DT(LQ_F16, false);
        else if (out_dtype == LQ_BF16) LQ_DECODE_DT(LQ_BF16, false);
        else LQ_DECODE_DT(LQ_F32, false);
    }
#undef LQ_DECODE_DT
#undef LQ_DECODE
#undef LQ_DECODE_E
    return launch_status();
}

int lq_chunk_decode(const uint32_t* d_words, const int64_t* d_chunk_base, const int64_t* d_stream_woff,
                    const uint32_t* d_blk_off, const int64_t* d_stream_nbits, const uint16_t* d_blk_state,
                    const uint8_t* d_coset_bits, const uint32_t* d_blk_n1, const lq_table* d_tables,
                    const uint16_t* d_scale16, int64_t n_chunks, int64_t n_heads, int64_t bph, uint32_t* d_lut_work,
                    void* d_out, int out_dtype, const int64_t* d_dither_seed, hipStream_t s) {
    (void)d_blk_n1;   // the decoder counts each block's coset-1 vectors from the bitmap
    return chunk_decode_launch(d_words, d_chunk_base, d_stream_woff, d_blk_off, d_stream_nbits, d_blk_state,
                               d_coset_bits, d_tables, d_scale16, n_chunks, n_heads, bph, d_lut_work, d_out, out_dtype,
                               d_dither_seed, 0, nullptr, nullptr, nullptr, nullptr, s);
}

int lq_chunk_decode_escaped(const uint32_t* d_words, const int64_t* d_chunk_base, const int64_t* d_stream_woff,
                            const uint32_t* d_blk_off, const int64_t* d_stream_nbits, const uint16_t* d_blk_state,
                            const uint8_t* d_coset_bits, const lq_table* d_tables, const uint16_t* d_scale16,
                            int64_t n_chunks, int64_t n_heads, int64_t bph, int head_dim, const float* d_signs,
                            const int32_t* d_esc_k, const int64_t* d_fine_off, const uint32_t* d_fine,
                            uint32_t* d_lut_work, void* d_out, int out_dtype, const int64_t* d_dither_seed, hipStream_t s) {
    if (!d_esc_k || !d_fine_off || !d_fine) return LQ_ERR_ARG;
    if (d_signs && (head_dim < 8 || head_dim > 128 || (head_dim & (head_dim - 1)) || bph <= 0 || bph % (head_dim / 8)))
        return LQ_ERR_ARG;
    return chunk_decode_launch(d_words, d_chunk_base, d_stream_woff, d_blk_off, d_stream_nbits, d_blk_state,
                               d_coset_bits, d_tables, d_scale16, n_chunks, n_heads, bph, d_lut_work, d_out, out_dtype,
                               d_dither_seed, d_signs ? head_dim : 0, d_signs, d_esc_k, d_fine_off, d_fine, s);
}

int lq_chunk_decode_rht(const uint32_t* d_words, const int64_t* d_chunk_base, const int64_t* d_stream_woff,
                        const uint32_t* d_blk_off, const int64_t* d_stream_nbits, const uint16_t* d_blk_state,
                        const uint8_t* d_coset_bits, const lq_table* d_tables, const uint16_t* d_scale16,
                        int64_t n_chunks, int64_t n_heads, int64_t bph, int head_dim, const float* d_signs,
                        uint32_t* d_lut_work, void* d_out, int out_dtype, const int64_t* d_dither_seed, hipStream_t s) {
    if (!d_signs || head_dim < 8 || head_dim > 128 || (head_dim & (head_dim - 1)) || bph <= 0 || bph % (head_dim / 8))
        return LQ_ERR_ARG;
    return chunk_decode_launch(d_words, d_chunk_base, d_stream_woff, d_blk_off, d_stream_nbits, d_blk_state,
                               d_coset_bits, d_tables, d_scale16, n_chunks, n_heads, bph, d_lut_work, d_out, out_dtype,
                               d_dither_seed, head_dim, d_signs, nullptr, nullptr, nullptr, s);
}

int lq_chunk_luts(const lq_table* d_tables, int64_t n_chunks, uint32_t* d_lut, hipStream_t s) {
    if (n_chunks <= 0 || !d_tables || !d_lut) return LQ_ERR_ARG;
    hipLaunchKernelGGL(k_chunk_lut, dim3((unsigned)(n_chunks * LQ_STREAMS)), dim3(256), 0, s, d_tables, d_lut, 0);
    return launch_status();
}

int lq_build_tables(const int64_t* d_counts, const int64_t* d_count_off, const int32_t* d_n_sym, int32_t n_tables,
                    int32_t* d_freqs, int32_t* d_cum, int32_t* d_lookup, int32_t* d_status, hipStream_t s) {
    if (n_tables <= 0) return LQ_ERR_ARG;
    hipLaunchKernelGGL(k_build_tables, dim3((unsigned)n_tables), dim3(256), 0, s, d_counts, d_count_off, d_n_sym, d_freqs,
                       d_cum, d_lookup, d_status);
    return launch_status();
}

int lq_rans_encode_streams(const int32_t* d_idx, const int64_t* d_sym_off, const int64_t* d_n, const int32_t* d_freqs,
                           const int32_t* d_cum, const int64_t* d_tab_off, int32_t n_streams, uint32_t* d_scratch,
                           uint32_t* d_words, const int64_t* d_word_off, int64_t* d_state, int64_t* d_nbits,
                           hipStream_t s) {
    if (n_streams <= 0) return LQ_ERR_ARG;
    hipLaunchKernelGGL(k_encode_streams, dim3((unsigned)((n_streams + 63) / 64)), dim3(64), 0, s, d_idx, d_sym_off, d_n,
                       d_freqs, d_cum, d_tab_off, n_streams, d_scratch, d_words, d_word_off, d_state, d_nbits);
    return launch_status();
}

int lq_rans_decode_streams(const int32_t* d_bits, const int32_t* d_bit_off, const int32_t* d_nbits, const int32_t* d_init,
                           const int32_t* d_ndec, const int32_t* d_lookup, const int32_t* d_freqs, const int32_t* d_cum,
                           const int32_t* d_alphabet, const int32_t* d_tid, int32_t max_sym, const int32_t* d_out_off,
                           int32_t n_streams, int64_t* d_out, hipStream_t s) {
    if (n_streams <= 0 || max_sym <= 0) return LQ_ERR_ARG;
    hipLaunchKernelGGL(k_decode_streams, dim3((unsigned)((n_streams + 63) / 64)), dim3(64), 0, s, d_bits, d_bit_off, d_nbits,
                       d_init, d_ndec, d_lookup, d_freqs, d_cum, d_alphabet, d_tid, max_sym, d_out_off, n_streams, d_out);
    return launch_status();
}

}  // extern "C"
