// Compressed decode attention for gfx950: one decode step of
// softmax(q K^T / sqrt(hd)) V where K and V are the E8 + rANS compressed
// prefix (chunks as lq_chunk_encode writes them, the reference's bitstreams)
// joined with an fp16 residual tail.
//
// Launches (after the K decoder LUTs):
//   k_attn_scores   K chunks -> partial scores S_c[qh][t] = sum over the
//                   coset-c dimensions of q[qh] . k[t], straight from the
//                   bitstreams (block-phase decoding, lq_decode.h); k is the
//                   fp16 value _decompress_chunk produces (lattice point times
//                   the fp16-stored scale, rounded to fp16).
//   lq_chunk_decode V chunks -> fp16 V, the cache the reference keeps resident.
//   k_attn_pv       split-token softmax . V: per (kv head, 512-token split of
//                   the prefix or of the fp16 tail), a record (m, l, o) per
//                   q head of the group.
//   k_attn_combine  log-sum-exp merge of a q head's records.
// head_dim is 128 (16 vectors per token); tokens per chunk are a multiple of
// 32 so that checkpoint blocks hold whole tokens of one head.
#include <climits>
#include <cmath>

#include "lq_decode.h"

using namespace lq;

namespace {

inline int launch_status() { return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_LAUNCH; }

constexpr int kHd = 128;
constexpr int kVpt = kHd / 8;            // vectors per token
constexpr int kTpb = kBlk / kVpt;        // tokens per block (32)
constexpr int kSB = 32;                  // blocks per scores workgroup (x 8 lanes = 256 threads)
constexpr int kSLanes = kSB * 8;
constexpr int kStgRowA = 72;             // u16 per block of the staging (8 x 8 + 8 padding)
constexpr int kSplit = 512;              // prefix tokens per k_attn_pv workgroup

template <int G>
__host__ __device__ constexpr int kQRow() { return 8 * G + 4; }

// Value of lane - d (d = 1, 2, 4) within the 16-lane row (DPP row_shr); lanes
// whose source leaves the row keep their own value.
__device__ __forceinline__ int dpp_shr(int v, int d) {
    switch (d) {
        case 1: return __builtin_amdgcn_update_dpp(v, v, 0x111, 0xf, 0xf, false);
        case 2: return __builtin_amdgcn_update_dpp(v, v, 0x112, 0xf, 0xf, false);
        default: return __builtin_amdgcn_update_dpp(v, v, 0x114, 0xf, 0xf, false);
    }
}
// Value of lane + 1 within the 16-lane row (DPP row_shl:1).
__device__ __forceinline__ int dpp_shl1(int v) { return __builtin_amdgcn_update_dpp(v, v, 0x101, 0xf, 0xf, false); }

struct BatchArgs {                        // device pointers of one chunk batch
    const uint32_t* words;
    const int64_t* chunk_base;
    const int64_t* stream_woff;
    const uint32_t* blk_off;
    const int64_t* stream_nbits;
    const uint16_t* blk_state;
    const uint8_t* coset_bits;
    const uint32_t* blk_n1;
    const lq_table* tables;
    const uint16_t* scale16;
    const uint32_t* lut;                  // k_chunk_lut output, n_chunks * 16 * L
    int64_t n_chunks, n_heads, bph, nblk;
};

// ------------------------------------------------------------ scores ----
// Workgroup: (chunk, coset c, head, group of up to 32 blocks of that head),
// lane (block b, coordinate idx).  After each 8-step phase lane idx rebuilds
// the phase's vector idx (fp16-rounded values), dots it with the q slice of
// its position in the token for the G q heads, and accumulates the partial
// per token in registers; a token change adds the partials into the LDS
// score tile.  S layout: S_c[qh][c_chunk * T + t], qh = head * G + j.
template <int G>
__global__ __launch_bounds__(256) void k_attn_scores(BatchArgs a, const uint16_t* __restrict__ q, float* __restrict__ S0,
                                                     float* __restrict__ S1) {
    __shared__ uint32_t lut[8 * kL];
    __shared__ uint32_t ring[kRing][kSLanes];
    __shared__ __align__(16) uint16_t stg[kSB * kStgRowA];
    __shared__ uint32_t bm[kSB][kBlk / 32 + 1];
    // q of the G heads by (slot in token, coordinate, head), slot rows padded by 16 bytes
    // so that lanes reading different slots hit different LDS banks
    __shared__ __align__(16) float qs[kVpt][kQRow<G>()];
    __shared__ float sp[kSB * kTpb][G];    // this coset's partial scores of the group's tokens
    const int tid = threadIdx.x;
    // blockIdx.x -> (chunk, coset, head, group)
    const int64_t bpHead = a.bph / kBlk;
    const int64_t gph = (bpHead + kSB - 1) / kSB;
    int64_t r = blockIdx.x;
    const int64_t gi = r % gph; r /= gph;
    const int64_t head = r % a.n_heads; r /= a.n_heads;
    const int c = (int)(r % 2);
    const int64_t chunk = r / 2;
    const int64_t g0 = head * bpHead + gi * kSB;        // first block (chunk-relative)
    const int nb = (int)(bpHead - gi * kSB < kSB ? bpHead - gi * kSB : kSB);
    const lq_table* T = a.tables + chunk * LQ_STREAMS + c * 8;
    const bool present = T[0].n_sym != 0;
    // LUTs and coset bitmaps (blocks are full: bph is a multiple of the block size)
    if (present) {
        const uint4* src = reinterpret_cast<const uint4*>(a.lut + (chunk * LQ_STREAMS + c * 8) * kL);
        uint4* dst = reinterpret_cast<uint4*>(lut);
        for (int i = tid; i < 8 * kL / 4; i += kSLanes) dst[i] = src[i];
        for (int i = tid; i < kSB * (kBlk / 32); i += kSLanes) {
            const int b = i / (kBlk / 32), w = i % (kBlk / 32);
            uint32_t m = 0;
            if (b < nb) {
                m = reinterpret_cast<const uint32_t*>(a.coset_bits + (chunk * a.nblk + g0 + b) * (kBlk / 8))[w];
                if (!c) m = ~m;
            }
            bm[b][w] = m;
        }
        for (int i = tid; i < kSB; i += kSLanes) bm[i][kBlk / 32] = 0u;
    }
    for (int i = tid; i < kHd * G; i += kSLanes) {
        const int d = i / G, j = i % G;
        qs[d / 8][(d % 8) * G + j] = h2f(q[(head * G + j) * kHd + d]);
    }
    for (int i = tid; i < kSB * kTpb * G; i += kSLanes) (&sp[0][0])[i] = 0.f;
    __syncthreads();

    const int b = tid >> 3, idx = tid & 7;
    const int64_t g = g0 + b;
    const int st = c * 8 + idx;
    const int64_t sid = chunk * LQ_STREAMS + st;
    const int64_t task = sid * a.nblk + g;
    int n = 0;
    if (present && b < nb) {
        const uint32_t n1 = a.blk_n1[chunk * a.nblk + g];
        n = c ? (int)n1 : kBlk - (int)n1;
    }
    if (n > 0) {
        CosetConsts cc;
        cc.init(T, c);
        const uint16_t s16 = a.scale16[chunk * a.n_heads + head];
        const float sc = h2f(s16);
        const _Float16 sh = __builtin_bit_cast(_Float16, s16);
        const half2_t sc2 = half2_t{sh, sh};
        PhaseLane<kSLanes> d;
        const int64_t end_bit = g + 1 < a.nblk ? (int64_t)a.blk_off[task + 1] : a.stream_nbits[sid];
        d.init(a.words + a.chunk_base[chunk] + a.stream_woff[sid], a.blk_off[task], end_bit, a.blk_state[task], lut, idx,
               &ring[0][tid], bm[b]);
        const char* const lutb = reinterpret_cast<const char*>(lut);
        uint16_t* const my_stg = &stg[b * kStgRowA + idx];
        for (int s0 = 0; s0 < n; s0 += kPhase) {
            d.boundary();
            const int m = n - s0 < kPhase ? n - s0 : kPhase;
            const int vl = d.phase(m, idx, my_stg, lutb);
            // lane idx: partial q . k of the vector of step idx, for the G heads
            float p[G];
            int t = INT_MAX;
#pragma unroll
            for (int j = 0; j < G; j++) p[j] = 0.f;
            if (idx < m) {
                const uint4 rr = *reinterpret_cast<const uint4*>(&stg[b * kStgRowA + idx * 8]);
                float y[8];
                if (cc.small) {
                    const uint4 h = cc.deq_f16(rr, sc2);
                    const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
                    for (int i = 0; i < 8; i++) y[i] = h2f((uint16_t)(hw[i >> 1] >> (16 * (i & 1))));
                } else {
                    cc.deq_f32(rr, sc, y);
#pragma unroll
                    for (int i = 0; i < 8; i++) y[i] = h2f(f2h(y[i]));
                }
                t = vl / kVpt;
                const float* qrow = &qs[vl % kVpt][0];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if constexpr (G == 4) {
                        const float4 qv = *reinterpret_cast<const float4*>(qrow + 4 * i);
                        p[0] = __builtin_fmaf(qv.x, y[i], p[0]);
                        p[1] = __builtin_fmaf(qv.y, y[i], p[1]);
                        p[2] = __builtin_fmaf(qv.z, y[i], p[2]);
                        p[3] = __builtin_fmaf(qv.w, y[i], p[3]);
                    } else {
#pragma unroll
                        for (int j = 0; j < G; j++) p[j] = __builtin_fmaf(qrow[i * G + j], y[i], p[j]);
                    }
                }
            }
            // the 8 lanes hold consecutive coset vectors (tokens ascending): a
            // segmented inclusive scan by token, then each segment's last lane
            // adds its token's sum (one writer per (block, token))
#pragma unroll
            for (int dd = 1; dd < 8; dd <<= 1) {
                const int ts = dpp_shr(t, dd);
                const bool take = idx >= dd && ts == t;
#pragma unroll
                for (int j = 0; j < G; j++) {
                    const float ps_ = __int_as_float(dpp_shr(__float_as_int(p[j]), dd));
                    p[j] = take ? p[j] + ps_ : p[j];
                }
            }
            const int tn = dpp_shl1(t);
            if (idx < m && (idx == 7 || tn != t)) {
#pragma unroll
                for (int j = 0; j < G; j++) sp[b * kTpb + t][j] += p[j];
            }
        }
    }
    __syncthreads();
    // coalesced store of the group's partial scores (zeros for an empty coset)
    const int64_t Tc = a.bph / kVpt;                       // tokens per head per chunk
    const int64_t row = a.n_chunks * Tc;
    const int64_t t0 = gi * kSB * kTpb;                    // first token of the group in the head
    float* Sc = c ? S1 : S0;
    for (int i = tid; i < nb * kTpb * G; i += kSLanes) {
        const int j = i / (nb * kTpb), tt = i % (nb * kTpb);
        Sc[(head * G + j) * row + chunk * Tc + t0 + tt] = sp[tt][j];
    }
}

// ------------------------------------------------------------ values ----
// Record per (kv head, split): m[G], l[G], o[G][kHd] with
// o = sum_t exp(s_t - m) v_t and l = sum_t exp(s_t - m) over the split.
template <int G>
__host__ __device__ constexpr int rec_floats() { return 2 * G + G * kHd; }

// Workgroup: (kv head, split); splits 0 .. n_split-1 cover 512 prefix tokens
// each (prefix token p is token p % Tc of chunk p / Tc), the next
// n_tsplit splits 512 tail tokens each.  Thread (token group tg = tid / 16,
// slice ds = tid % 16) owns dimensions 8 ds .. 8 ds + 7 of tokens tg,
// tg + 16, ..: one 16-byte load per token, eight tokens in flight.
template <int G>
__global__ __launch_bounds__(256) void k_attn_pv(const float* __restrict__ S0, const float* __restrict__ S1,
                                                 const uint16_t* __restrict__ vdec, int64_t n_chunks, int64_t n_heads,
                                                 int64_t Tc, int64_t n_split, int64_t n_tsplit,
                                                 const uint16_t* __restrict__ q, const uint16_t* __restrict__ tail_k,
                                                 const uint16_t* __restrict__ tail_v, int64_t t_tail, float qk_scale,
                                                 float* __restrict__ rec) {
    __shared__ float ps[kSplit][G];   // scores, then weights
    __shared__ float qv[G][kHd];
    __shared__ float red[4][G];
    __shared__ float mx[G], sm[G];
    __shared__ float ow[4][G][kHd];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tg = tid >> 4, ds = tid & 15;
    const int64_t n_rec = n_split + n_tsplit;
    const int64_t head = blockIdx.x / n_rec;
    const int64_t split = blockIdx.x % n_rec;
    const bool is_tail = split >= n_split;
    const int64_t row = n_chunks * Tc;
    const int64_t tb = is_tail ? (split - n_split) * kSplit : split * kSplit;
    const int64_t lim = is_tail ? t_tail : row;
    const int ntok = (int)(lim - tb < kSplit ? lim - tb : kSplit);
    float* rr = rec + blockIdx.x * (int64_t)rec_floats<G>();
    // prefix token tb + t is token tt0 + t of chunk ch0 while tt0 + t < Tc (one division per workgroup)
    const int64_t ch0 = is_tail ? 0 : tb / Tc;
    const int tt0 = is_tail ? 0 : (int)(tb - ch0 * Tc);
    auto vrow = [&](const uint16_t* base, int t) -> const uint4* {
        if (is_tail) return reinterpret_cast<const uint4*>(base + (head * t_tail + tb + t) * kHd) + ds;
        int64_t ch = ch0;
        int tt = tt0 + t;
        while (tt >= Tc) { tt -= (int)Tc; ch++; }
        return reinterpret_cast<const uint4*>(base + ((ch * n_heads + head) * Tc + tt) * kHd) + ds;
    };
    auto unpack8 = [](const uint4& vv, float v[8]) {
        const uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = h2f((uint16_t)(w4[k >> 1] >> (16 * (k & 1))));
    };
    const uint16_t* vsrc = is_tail ? tail_v : vdec;
    // scores of the split's tokens
    if (is_tail) {
        for (int i = tid; i < G * kHd; i += 256) qv[i / kHd][i % kHd] = h2f(q[(head * G) * kHd + i]);
        __syncthreads();
        for (int t0 = 0; t0 < ntok; t0 += 16) {   // the 16 lanes of a token group share a token
            const int t = t0 + tg;
            float kf[8];
            if (t < ntok) unpack8(*vrow(tail_k, t), kf);
            else {
#pragma unroll
                for (int k = 0; k < 8; k++) kf[k] = 0.f;
            }
#pragma unroll
            for (int j = 0; j < G; j++) {
                float part = 0.f;
#pragma unroll
                for (int k = 0; k < 8; k++) part = __builtin_fmaf(qv[j][ds * 8 + k], kf[k], part);
                part += __shfl_xor(part, 8, 16);
                part += __shfl_xor(part, 4, 16);
                part += __shfl_xor(part, 2, 16);
                part += __shfl_xor(part, 1, 16);
                if (ds == 0 && t < ntok) ps[t][j] = part * qk_scale;
            }
        }
    } else {
        // all loads of the split's scores first, then the LDS writes
        constexpr int kPer = (kSplit * G + 255) / 256;
        float a0[kPer], a1[kPer];
#pragma unroll
        for (int u = 0; u < kPer; u++) {
            const int i = tid + 256 * u;
            const int j = i / ntok, t = i % ntok;
            const int64_t o = (head * G + j) * row + tb + t;
            a0[u] = i < ntok * G ? S0[o] : 0.f;
            a1[u] = i < ntok * G ? S1[o] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kPer; u++) {
            const int i = tid + 256 * u;
            if (i < ntok * G) ps[i % ntok][i / ntok] = (a0[u] + a1[u]) * qk_scale;
        }
    }
    __syncthreads();
    // max and weights per q head
#pragma unroll
    for (int j = 0; j < G; j++) {
        float m = -INFINITY;
        for (int t = tid; t < ntok; t += 256) m = fmaxf(m, ps[t][j]);
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (lane == 0) red[wave][j] = m;
    }
    __syncthreads();
    if (tid < G) mx[tid] = fmaxf(fmaxf(red[0][tid], red[1][tid]), fmaxf(red[2][tid], red[3][tid]));
    __syncthreads();
#pragma unroll
    for (int j = 0; j < G; j++) {
        const float mj = mx[j];
        float ssum = 0.f;
        for (int t = tid; t < ntok; t += 256) {
            const float e = __expf(ps[t][j] - mj);
            ps[t][j] = e;
            ssum += e;
        }
        for (int o = 32; o > 0; o >>= 1) ssum += __shfl_xor(ssum, o, 64);
        if (lane == 0) red[wave][j] = ssum;
    }
    __syncthreads();
    if (tid < G) sm[tid] = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
    float o[G][8];
#pragma unroll
    for (int j = 0; j < G; j++)
#pragma unroll
        for (int k = 0; k < 8; k++) o[j][k] = 0.f;
    auto accum = [&](int t, const uint4& vv) {
        float v[8];
        unpack8(vv, v);
#pragma unroll
        for (int j = 0; j < G; j++) {
            const float pj = ps[t][j];
#pragma unroll
            for (int k = 0; k < 8; k++) o[j][k] = __builtin_fmaf(pj, v[k], o[j][k]);
        }
    };
    int t = tg;
    for (; t + 112 < ntok; t += 128) {   // 8 loads in flight
        uint4 a[8];
#pragma unroll
        for (int u = 0; u < 8; u++) a[u] = *vrow(vsrc, t + 16 * u);
#pragma unroll
        for (int u = 0; u < 8; u++) accum(t + 16 * u, a[u]);
    }
    for (; t < ntok; t += 16) accum(t, *vrow(vsrc, t));
    // reduce the 16 token groups: 4 per wave by shuffles, then the 4 waves through LDS
#pragma unroll
    for (int j = 0; j < G; j++)
#pragma unroll
        for (int k = 0; k < 8; k++) {
            float x = o[j][k];
            x += __shfl_xor(x, 16, 64);
            x += __shfl_xor(x, 32, 64);
            o[j][k] = x;
        }
    if (lane < 16) {
#pragma unroll
        for (int j = 0; j < G; j++)
#pragma unroll
            for (int k = 0; k < 8; k++) ow[wave][j][ds * 8 + k] = o[j][k];
    }
    __syncthreads();
    for (int i = tid; i < G * kHd; i += 256) {
        const int j = i / kHd, dd = i % kHd;
        rr[2 * G + i] = (ow[0][j][dd] + ow[1][j][dd]) + (ow[2][j][dd] + ow[3][j][dd]);
    }
    if (tid < G) {
        rr[tid] = mx[tid];
        rr[G + tid] = sm[tid];
    }
}

// ----------------------------------------------------------- combine ----
// One workgroup of 128 threads per q head: log-sum-exp merge of its kv
// head's records (a record with m = -inf weighs nothing); thread d owns
// output dimension d.
constexpr int kMaxW = 2048;   // record weights kept in LDS; more are recomputed

template <int G>
__global__ __launch_bounds__(128) void k_attn_combine(const float* __restrict__ rec, int64_t n_rec,
                                                      uint16_t* __restrict__ out) {
    __shared__ float w[kMaxW];
    __shared__ float red[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t qh = blockIdx.x;
    const int64_t head = qh / G;
    const int j = (int)(qh % G);
    const float* r0 = rec + head * n_rec * rec_floats<G>();
    float m = -INFINITY;
    for (int64_t r = tid; r < n_rec; r += 128) m = fmaxf(m, r0[r * rec_floats<G>() + j]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(red[0], red[1]);
    __syncthreads();
    auto weight = [&](int64_t r) {
        const float mr = r0[r * rec_floats<G>() + j];
        return mr == -INFINITY ? 0.f : __expf(mr - m);
    };
    float l = 0.f;
    for (int64_t r = tid; r < n_rec; r += 128) {
        const float e = weight(r);
        if (r < kMaxW) w[r] = e;
        l = __builtin_fmaf(r0[r * rec_floats<G>() + G + j], e, l);
    }
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
    if (lane == 0) red[wave] = l;
    __syncthreads();
    l = red[0] + red[1];
    __syncthreads();
    float acc = 0.f;
    int64_t r = 0;
    for (; r + 8 <= n_rec; r += 8) {   // 8 record loads in flight
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; u++) x[u] = r0[(r + u) * rec_floats<G>() + 2 * G + j * kHd + tid];
#pragma unroll
        for (int u = 0; u < 8; u++) acc = __builtin_fmaf(x[u], r + u < kMaxW ? w[r + u] : weight(r + u), acc);
    }
    for (; r < n_rec; r++) acc = __builtin_fmaf(r0[r * rec_floats<G>() + 2 * G + j * kHd + tid],
                                                r < kMaxW ? w[r] : weight(r), acc);
    out[qh * kHd + tid] = f2h(acc / l);
}

struct AttnWork {
    int64_t lut_k, lut_v, s0, s1, vdec, rec, total;
};

__host__ inline AttnWork attn_layout(int64_t n_chunks, int64_t n_heads, int64_t bph, int G) {
    AttnWork w;
    const int64_t T = bph / kVpt;
    const int64_t n_split = (n_chunks * T + kSplit - 1) / kSplit;
    const int64_t n_tsplit = (1024 + kSplit - 1) / kSplit;   // records reserved for the largest tail
    auto al = [](int64_t b) { return ((b + 255) / 256) * 256; };
    w.lut_k = 0;
    w.lut_v = al(w.lut_k + n_chunks * LQ_STREAMS * kL * 4);
    w.s0 = al(w.lut_v + n_chunks * LQ_STREAMS * kL * 4);
    w.s1 = al(w.s0 + n_heads * G * n_chunks * T * 4);
    w.vdec = al(w.s1 + n_heads * G * n_chunks * T * 4);
    w.rec = al(w.vdec + n_chunks * n_heads * bph * 8 * 2);
    w.total = al(w.rec + n_heads * (n_split + n_tsplit) * (int64_t)(2 * G + G * kHd) * 4);
    return w;
}

BatchArgs to_args(const lq_chunk_batch* b, const uint32_t* lut) {
    BatchArgs a;
    a.words = b->words;
    a.chunk_base = b->chunk_base;
    a.stream_woff = b->stream_woff;
    a.blk_off = b->blk_off;
    a.stream_nbits = b->stream_nbits;
    a.blk_state = b->blk_state;
    a.coset_bits = b->coset_bits;
    a.blk_n1 = b->blk_n1;
    a.tables = b->tables;
    a.scale16 = b->scale16;
    a.lut = lut;
    a.n_chunks = b->n_chunks;
    a.n_heads = b->n_heads;
    a.bph = b->bph;
    a.nblk = (b->n_heads * b->bph + kBlk - 1) / kBlk;
    return a;
}

bool batch_ok(const lq_chunk_batch* b) {
    return b && b->words && b->tables && b->stream_nbits && b->n_chunks > 0 && b->n_heads > 0 && b->bph > 0 &&
           b->bph % (kTpb * kVpt) == 0;
}

}  // namespace

extern "C" {

int64_t lq_attn_workspace(int64_t n_chunks, int64_t n_heads, int64_t bph, int group) {
    if (n_chunks <= 0 || n_heads <= 0 || bph <= 0 || group <= 0) return -1;
    return attn_layout(n_chunks, n_heads, bph, group).total;
}

int lq_decode_attention(const lq_chunk_batch* k, const lq_chunk_batch* v, const uint16_t* d_q, int group,
                        const uint16_t* d_tail_k, const uint16_t* d_tail_v, int64_t t_tail, void* d_work,
                        uint16_t* d_out, hipStream_t s) {
    if (!batch_ok(k) || !batch_ok(v) || !d_q || !d_out || !d_work) return LQ_ERR_ARG;
    if (k->n_chunks != v->n_chunks || k->n_heads != v->n_heads || k->bph != v->bph) return LQ_ERR_ARG;
    if (group != 1 && group != 2 && group != 4 && group != 8) return LQ_ERR_ARG;
    if (t_tail < 0 || t_tail > 1024 || (t_tail > 0 && (!d_tail_k || !d_tail_v))) return LQ_ERR_ARG;
    const AttnWork w = attn_layout(k->n_chunks, k->n_heads, k->bph, group);
    char* base = reinterpret_cast<char*>(d_work);
    uint32_t* lut_k = reinterpret_cast<uint32_t*>(base + w.lut_k);
    uint32_t* lut_v = reinterpret_cast<uint32_t*>(base + w.lut_v);
    float* S0 = reinterpret_cast<float*>(base + w.s0);
    float* S1 = reinterpret_cast<float*>(base + w.s1);
    uint16_t* vdec = reinterpret_cast<uint16_t*>(base + w.vdec);
    float* rec = reinterpret_cast<float*>(base + w.rec);
    int rc = lq_chunk_luts(k->tables, k->n_chunks, lut_k, s);
    if (rc) return rc;
    // V: decode + dequantise to fp16 (n_chunks, n_heads, T, 128)
    rc = lq_chunk_decode(v->words, v->chunk_base, v->stream_woff, v->blk_off, v->stream_nbits, v->blk_state,
                         v->coset_bits, v->blk_n1, v->tables, v->scale16, v->n_chunks, v->n_heads, v->bph, lut_v, vdec,
                         LQ_F16, nullptr, s);
    if (rc) return rc;
    const BatchArgs ak = to_args(k, lut_k);
    const int64_t gph = ((k->bph / kBlk) + kSB - 1) / kSB;
    const dim3 grid((unsigned)(k->n_chunks * 2 * k->n_heads * gph));
    const float qk_scale = 1.0f / sqrtf((float)kHd);
    const int64_t Tc = k->bph / kVpt;
    const int64_t n_split = (k->n_chunks * Tc + kSplit - 1) / kSplit;
    const int64_t n_tsplit = (t_tail + kSplit - 1) / kSplit;
    const int64_t nq = k->n_heads * group;
#define LQ_ATTN(GG)                                                                                              \
    do {                                                                                                         \
        hipLaunchKernelGGL((k_attn_scores<GG>), grid, dim3(kSLanes), 0, s, ak, d_q, S0, S1);                     \
        hipLaunchKernelGGL((k_attn_pv<GG>), dim3((unsigned)(k->n_heads * (n_split + n_tsplit))), dim3(256), 0, s, \
                           S0, S1, vdec, k->n_chunks, k->n_heads, Tc, n_split, n_tsplit, d_q, d_tail_k, d_tail_v, \
                           t_tail, qk_scale, rec);                                                               \
        hipLaunchKernelGGL((k_attn_combine<GG>), dim3((unsigned)nq), dim3(kHd), 0, s, rec, n_split + n_tsplit,    \
                           d_out);                                                                               \
    } while (0)
    if (group == 1) LQ_ATTN(1);
    else if (group == 2) LQ_ATTN(2);
    else if (group == 4) LQ_ATTN(4);
    else LQ_ATTN(8);
#undef LQ_ATTN
    return launch_status();
}

}  // extern "C"
