// Fused compressed decode attention for gfx950: one decode step of
// softmax(q K^T / sqrt(hd)) V where K and V are the E8 + rANS compressed
// prefix (chunks as lq_chunk_encode writes them, the reference's bitstreams)
// joined with an fp16 residual tail.
//
// Three launches (after the per-chunk decoder LUTs):
//   k_attn_qk       K chunks -> scores S_c[qh][t] = sum_d q[qh][d] * k[t][d], one
//                   partial per coset (the coset's dimensions of each token).
//   k_attn_pv       V chunks: p = exp((S_0 + S_1) / sqrt(hd) - m_local),
//                   o_local = sum_t p v, one record (m, l, o) per
//                   (chunk, coset, head, 32-block group).
// k and v are the fp16 values _decompress_chunk produces (lattice point times
// the fp16-stored scale, rounded to fp16), so the step attends over exactly
// the cache the reference keeps resident.
//   k_attn_combine  log-sum-exp merge of the records and the fp16 tail per q head.
// Each workgroup of the two decode kernels owns one coset of up to 32 blocks
// (LQ_BLK vectors each) of one head: lane (block, coordinate) decodes its
// stream from the block checkpoint, the 8 lanes of a block run in lockstep on
// the coset's vectors (as k_chunk_decode does), so c7's parity comes from one
// wave ballot.  head_dim is 128 (16 vectors per token); tokens per chunk are a
// multiple of 32 so that blocks hold whole tokens of one head.
#include <cmath>

#include "lq_decode.h"

using namespace lq;

namespace {

inline int launch_status() { return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_LAUNCH; }

constexpr int kHd = 128;
constexpr int kVpt = kHd / 8;            // vectors per token
constexpr int kTpb = kBlk / kVpt;        // tokens per block (32)
constexpr int kGB = 32;                  // blocks per workgroup (x 8 lanes = 256 threads)

struct BatchArgs {                        // device pointers of one chunk batch
    const uint32_t* words;
    const int64_t* chunk_base;
    const int64_t* stream_woff;
    const uint32_t* blk_off;
    const uint16_t* blk_state;
    const uint8_t* coset_bits;
    const uint32_t* blk_n1;
    const lq_table* tables;
    const uint16_t* scale16;
    const uint32_t* lut;                  // k_chunk_lut output, n_chunks * 16 * L
    int64_t n_chunks, n_heads, bph, nblk;
};

// Workgroup geometry shared by the two decode kernels: blockIdx.x ->
// (chunk, coset, head, group of kGB blocks inside the head).
struct WgPos {
    int64_t chunk, head, g0;   // g0: first block (chunk-relative)
    int c, nb;                 // coset, blocks in this workgroup
};

__device__ __forceinline__ WgPos wg_pos(const BatchArgs& a) {
    const int64_t bpHead = a.bph / kBlk;
    const int64_t gph = (bpHead + kGB - 1) / kGB;   // groups per head
    int64_t r = blockIdx.x;
    WgPos p;
    const int64_t gi = r % gph; r /= gph;
    p.head = r % a.n_heads; r /= a.n_heads;
    p.c = (int)(r % 2);
    p.chunk = r / 2;
    p.g0 = p.head * bpHead + gi * kGB;
    const int64_t left = bpHead - gi * kGB;
    p.nb = (int)(left < kGB ? left : kGB);
    return p;
}

// One lane's decoder of stream (coset c, coordinate idx) inside block g:
// StreamDec (lq_decode.h) plus the walk over the block's coset bitmap that
// yields each symbol's vector index.
struct LaneDecoder {
    StreamDec d;
    const uint32_t* LU;   // the LDS block of the coset's 8 LUTs
    int lo_sym, ncnt, steps;
    // coset-c vectors of the block, ascending, from the LDS bitmap
    const uint32_t* bm;
    int c, wi;
    uint32_t wv;

    __device__ __forceinline__ uint32_t word_of(int w) const {
        uint32_t m = bm[w];
        return c ? m : ~m;   // blocks are full (LQ_BLK vectors): no tail mask
    }

    __device__ __forceinline__ void init(const BatchArgs& a, int64_t chunk, int64_t g, int c_, int idx,
                                         const uint32_t* lut_lds, const uint32_t* bm_lds) {
        c = c_;
        bm = bm_lds;
        const int st = c * 8 + idx;
        const int64_t task = (chunk * LQ_STREAMS + st) * a.nblk + g;
        const uint32_t n1 = a.blk_n1[chunk * a.nblk + g];
        ncnt = c ? (int)n1 : kBlk - (int)n1;
        lo_sym = a.tables[chunk * LQ_STREAMS + st].lo;
        LU = lut_lds;
        steps = 0;
        if (ncnt > 0)
            d.init(a.words + a.chunk_base[chunk] + a.stream_woff[chunk * LQ_STREAMS + st], a.blk_off[task],
                   a.blk_state[task], LU, idx);
        wi = 0;
        wv = word_of(0);
    }

    // Next symbol value (alphabet value, before parity) and its vector index.
    __device__ __forceinline__ int next(int* vl) {
        if (steps % 3 == 0) d.refill();
        steps++;
        const int val = lo_sym + (int)d.sym();
        d.step(LU);
        while (wv == 0) wv = word_of(++wi);
        *vl = 32 * wi + __builtin_ctz(wv);
        wv &= wv - 1u;
        return val;
    }
};

// Dequantised value of the symbol a lane just decoded, as _decompress_chunk
// produces it: fp16((coordinate + coset offset) * scale16), widened.
// Coordinate 7 is 2 * val + parity(c0 + .. + c6), the parity from the low
// bits of the 8-lane group's symbols.
__device__ __forceinline__ float coord_value(int val, int idx, int c, bool active, float sc) {
    const unsigned long long odd = __ballot(active && (val & 1));
    const int par = __popcll(odd & (0x7full << (threadIdx.x & 56))) & 1;
    const int coord = idx < 7 ? val : 2 * val + par;
    return h2f(f2h(((float)coord + (c ? 0.5f : 0.f)) * sc));
}

// Copy the coset's 8 decoder LUTs and the group's coset bitmap words to LDS.
__device__ __forceinline__ void stage_lut_bitmap(const BatchArgs& a, const WgPos& p, uint32_t (*lut)[kL],
                                                 uint32_t (*bm)[kBlk / 32]) {
    const int tid = threadIdx.x;
    const uint4* src = reinterpret_cast<const uint4*>(a.lut + (p.chunk * LQ_STREAMS + p.c * 8) * kL);
    uint4* dst = reinterpret_cast<uint4*>(&lut[0][0]);
    for (int i = tid; i < 8 * kL / 4; i += 256) dst[i] = src[i];
    for (int i = tid; i < kGB * (kBlk / 32); i += 256) {
        const int b = i / (kBlk / 32), w = i % (kBlk / 32);
        bm[b][w] = b < p.nb ? reinterpret_cast<const uint32_t*>(a.coset_bits + (p.chunk * a.nblk + p.g0 + b) * (kBlk / 8))[w]
                            : 0u;
    }
}

// ------------------------------------------------------------ scores ----
// S layout: S_c[qh][c_chunk * T + t], qh = head * G + j, row length n_chunks * T.
template <int G>
__global__ __launch_bounds__(256) void k_attn_qk(BatchArgs a, const uint16_t* __restrict__ q, float* __restrict__ S0,
                                                 float* __restrict__ S1) {
    __shared__ uint32_t lut[8][kL];
    __shared__ uint32_t bm[kGB][kBlk / 32];
    __shared__ float qs[kHd][G];
    __shared__ float sp[kGB * kTpb][G];   // this coset's partial scores of the group's tokens
    const int tid = threadIdx.x;
    const WgPos p = wg_pos(a);
    const lq_table* T = a.tables + p.chunk * LQ_STREAMS + p.c * 8;
    const bool present = T[0].n_sym != 0;
    if (present) stage_lut_bitmap(a, p, lut, bm);
    for (int i = tid; i < kHd * G; i += 256) {
        const int d = i / G, j = i % G;
        qs[d][j] = h2f(q[(p.head * G + j) * kHd + d]);
    }
    for (int i = tid; i < kGB * kTpb * G; i += 256) (&sp[0][0])[i] = 0.f;
    __syncthreads();
    const int b = tid >> 3, idx = tid & 7;
    const bool live = present && b < p.nb;
    const float sc = h2f(a.scale16[p.chunk * a.n_heads + p.head]);
    if (present) {
        LaneDecoder dec;
        if (live) dec.init(a, p.chunk, p.g0 + b, p.c, idx, &lut[0][0], bm[b]);
        const int n = live ? dec.ncnt : 0;
        // the 8 lanes of a block share n; loop to the wave's max so ballots see every lane
        int nmax = n;
        for (int o = 8; o < 64; o <<= 1) nmax = max(nmax, __shfl_xor(nmax, o, 64));
        // per-lane partial of the current token; on a token change the 8 lanes
        // of the block add theirs into the token's LDS slot (one instruction,
        // same-address lanes applied in hardware lane order)
        float acc[G];
#pragma unroll
        for (int j = 0; j < G; j++) acc[j] = 0.f;
        int cur_t = -1;
        for (int s = 0; s < nmax; s++) {
            const bool act = s < n;
            int vl = 0, val = 0;
            if (act) val = dec.next(&vl);
            const float v = coord_value(val, idx, p.c, act, sc);
            if (act) {
                const int t = vl / kVpt;
                if (t != cur_t && cur_t >= 0) {
#pragma unroll
                    for (int j = 0; j < G; j++) {
                        atomicAdd(&sp[b * kTpb + cur_t][j], acc[j]);
                        acc[j] = 0.f;
                    }
                }
                cur_t = t;
                const int d = (vl % kVpt) * 8 + idx;
#pragma unroll
                for (int j = 0; j < G; j++) acc[j] = __builtin_fmaf(qs[d][j], v, acc[j]);
            }
        }
        if (live && cur_t >= 0) {
#pragma unroll
            for (int j = 0; j < G; j++) atomicAdd(&sp[b * kTpb + cur_t][j], acc[j]);
        }
    }
    __syncthreads();
    // coalesced store of the group's partial scores (zeros for an empty coset)
    const int64_t Tc = a.bph / kVpt;                       // tokens per head per chunk
    const int64_t row = a.n_chunks * Tc;
    const int64_t t0 = (p.g0 - p.head * (a.bph / kBlk)) * kTpb;   // first token of the group in the head
    float* Sc = p.c ? S1 : S0;
    for (int i = tid; i < p.nb * kTpb * G; i += 256) {
        const int j = i / (p.nb * kTpb), tt = i % (p.nb * kTpb);
        Sc[(p.head * G + j) * row + p.chunk * Tc + t0 + tt] = sp[tt][j];
    }
}

// ------------------------------------------------------------ values ----
// Record per workgroup: m[G], l[G], o[G][kHd].
template <int G>
__host__ __device__ constexpr int rec_floats() { return 2 * G + G * kHd; }

template <int G>
__global__ __launch_bounds__(256) void k_attn_pv(BatchArgs a, const float* __restrict__ S0,
                                                 const float* __restrict__ S1, float qk_scale, float* __restrict__ rec) {
    __shared__ uint32_t lut[8][kL];
    __shared__ uint32_t bm[kGB][kBlk / 32];
    __shared__ float pw[kGB * kTpb][G];           // softmax weights of the group's tokens
    __shared__ float tb[kGB][kVpt][8];            // per 8-lane group: dequantised values of its current token
    __shared__ float red[4][G];
    __shared__ float mx[G], sm[G];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const WgPos p = wg_pos(a);
    const lq_table* T = a.tables + p.chunk * LQ_STREAMS + p.c * 8;
    const bool present = T[0].n_sym != 0;
    if (present) stage_lut_bitmap(a, p, lut, bm);
    for (int i = tid; i < kGB * kVpt * 8; i += 256) (&tb[0][0][0])[i] = 0.f;
    // scores -> local max / weights / sum
    const int64_t Tc = a.bph / kVpt;
    const int64_t row = a.n_chunks * Tc;
    const int64_t t0 = (p.g0 - p.head * (a.bph / kBlk)) * kTpb;
    const int ntok = p.nb * kTpb;
    const float sk = qk_scale;
    float lm[G];
#pragma unroll
    for (int j = 0; j < G; j++) lm[j] = -INFINITY;
    for (int i = tid; i < ntok * G; i += 256) {
        const int j = i / ntok, tt = i % ntok;
        const int64_t o = (p.head * G + j) * row + p.chunk * Tc + t0 + tt;
        const float s = (S0[o] + S1[o]) * sk;
        pw[tt][j] = s;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < G; j++) {
        float m = -INFINITY;
        for (int tt = tid; tt < ntok; tt += 256) m = fmaxf(m, pw[tt][j]);
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (lane == 0) red[wave][j] = m;
    }
    __syncthreads();
    if (tid < G) mx[tid] = fmaxf(fmaxf(red[0][tid], red[1][tid]), fmaxf(red[2][tid], red[3][tid]));
    __syncthreads();
#pragma unroll
    for (int j = 0; j < G; j++) {
        lm[j] = mx[j];
        float ssum = 0.f;
        for (int tt = tid; tt < ntok; tt += 256) {
            const float e = __expf(pw[tt][j] - lm[j]);
            pw[tt][j] = e;
            ssum += e;
        }
        for (int o = 32; o > 0; o >>= 1) ssum += __shfl_xor(ssum, o, 64);
        __syncthreads();
        if (lane == 0) red[wave][j] = ssum;
        __syncthreads();
        if (tid == 0) sm[j] = (red[0][j] + red[1][j]) + (red[2][j] + red[3][j]);
    }
    __syncthreads();

    const int b = tid >> 3, idx = tid & 7;
    const bool live = present && b < p.nb;
    const float sv = h2f(a.scale16[p.chunk * a.n_heads + p.head]);
    float o[G][kVpt];
#pragma unroll
    for (int j = 0; j < G; j++)
#pragma unroll
        for (int m = 0; m < kVpt; m++) o[j][m] = 0.f;
    if (present) {
        LaneDecoder dec;
        if (live) dec.init(a, p.chunk, p.g0 + b, p.c, idx, &lut[0][0], bm[b]);
        const int n = live ? dec.ncnt : 0;
        int nmax = n;
        for (int s = 8; s < 64; s <<= 1) nmax = max(nmax, __shfl_xor(nmax, s, 64));
        int cur_t = -1;
        float (*tok)[8] = tb[b];
        // apply the finished token: o[j][m] += p[t][j] * value(m, idx); clear the buffer
        auto flush = [&](int t) {
            float pj[G];
#pragma unroll
            for (int j = 0; j < G; j++) pj[j] = pw[b * kTpb + t][j];
#pragma unroll
            for (int m = 0; m < kVpt; m++) {
                const float v = tok[m][idx];
                tok[m][idx] = 0.f;
#pragma unroll
                for (int j = 0; j < G; j++) o[j][m] = __builtin_fmaf(pj[j], v, o[j][m]);
            }
        };
        for (int s = 0; s < nmax; s++) {
            const bool act = s < n;
            int vl = 0, val = 0;
            if (act) val = dec.next(&vl);
            const float v = coord_value(val, idx, p.c, act, sv);
            if (act) {
                const int t = vl / kVpt;
                if (t != cur_t && cur_t >= 0) flush(cur_t);
                cur_t = t;
                tok[vl % kVpt][idx] = v;
            }
        }
        if (live && cur_t >= 0) flush(cur_t);
    }
    // reduce o over the blocks: 8 groups per wave by shuffles, then the 4 waves through LDS
#pragma unroll
    for (int j = 0; j < G; j++)
#pragma unroll
        for (int m = 0; m < kVpt; m++) {
            float r = o[j][m];
            r += __shfl_xor(r, 8, 64);
            r += __shfl_xor(r, 16, 64);
            r += __shfl_xor(r, 32, 64);
            o[j][m] = r;
        }
    __syncthreads();
    float* ow = &tb[0][0][0];   // reuse: [4 waves][G][kHd] needs 4 * G * 128 floats <= kGB * kVpt * 8
    static_assert(4 * G * kHd <= kGB * kVpt * 8, "LDS reuse too small");
    if (lane < 8) {
#pragma unroll
        for (int j = 0; j < G; j++)
#pragma unroll
            for (int m = 0; m < kVpt; m++) ow[(wave * G + j) * kHd + m * 8 + lane] = o[j][m];
    }
    __syncthreads();
    float* r = rec + (int64_t)blockIdx.x * rec_floats<G>();
    for (int i = tid; i < G * kHd; i += 256)
        r[2 * G + i] = (ow[i] + ow[G * kHd + i]) + (ow[2 * G * kHd + i] + ow[3 * G * kHd + i]);
    if (tid < G) {
        r[tid] = mx[tid];
        r[G + tid] = sm[tid];
    }
}

// ----------------------------------------------------------- combine ----
// One workgroup per q head: merge the records of its kv head (both cosets of
// every chunk group; m and l are the same in the two coset records) with the
// fp16 tail tokens, write fp16 o / l.
template <int G>
__global__ __launch_bounds__(256) void k_attn_combine(const float* __restrict__ rec, int64_t n_chunks, int64_t n_heads,
                                                      int64_t gph, const uint16_t* __restrict__ q,
                                                      const uint16_t* __restrict__ tail_k,
                                                      const uint16_t* __restrict__ tail_v, int64_t t_tail,
                                                      float qk_scale, uint16_t* __restrict__ out) {
    __shared__ float qv[kHd];
    __shared__ float ts[1024];
    __shared__ float red[4];
    __shared__ float s_m;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t qh = blockIdx.x;
    const int64_t head = qh / G;
    const int j = (int)(qh % G);
    if (tid < kHd) qv[tid] = h2f(q[qh * kHd + tid]);
    __syncthreads();
    // global max over record maxima and tail scores
    const int64_t nrec = n_chunks * gph;   // per coset
    auto rec_at = [&](int64_t chunk, int c, int64_t gi) {
        return rec + (((chunk * 2 + c) * n_heads + head) * gph + gi) * rec_floats<G>();
    };
    float m = -INFINITY;
    for (int64_t r = tid; r < nrec; r += 256) m = fmaxf(m, rec_at(r / gph, 0, r % gph)[j]);
    const int64_t ntail = t_tail < 1024 ? t_tail : 1024;
    for (int64_t t = tid; t < ntail; t += 256) {
        const uint16_t* kt = tail_k + (head * t_tail + t) * kHd;
        float s = 0.f;
        for (int d = 0; d < kHd; d++) s = __builtin_fmaf(qv[d], h2f(kt[d]), s);
        s *= qk_scale;
        ts[t] = s;
        m = fmaxf(m, s);
    }
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    if (tid == 0) s_m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    m = s_m;
    // l and o: thread d < 128 accumulates output dimension d
    float l = 0.f, acc = 0.f;
    if (tid < kHd) {
        for (int64_t r = 0; r < nrec; r++) {
            const float* r0 = rec_at(r / gph, 0, r % gph);
            const float* r1 = rec_at(r / gph, 1, r % gph);
            const float w = __expf(r0[j] - m);
            l = __builtin_fmaf(r0[G + j], w, l);
            acc = __builtin_fmaf(r0[2 * G + j * kHd + tid] + r1[2 * G + j * kHd + tid], w, acc);
        }
        for (int64_t t = 0; t < ntail; t++) {
            const float w = __expf(ts[t] - m);
            l += w;
            acc = __builtin_fmaf(w, h2f(tail_v[(head * t_tail + t) * kHd + tid]), acc);
        }
        out[qh * kHd + tid] = f2h(acc / l);
    }
}

struct AttnWork {
    int64_t lut_k, lut_v, s0, s1, rec, total;
};

__host__ inline AttnWork attn_layout(int64_t n_chunks, int64_t n_heads, int64_t bph, int G) {
    AttnWork w;
    const int64_t T = bph / kVpt;
    const int64_t gph = ((bph / kBlk) + kGB - 1) / kGB;
    auto al = [](int64_t b) { return ((b + 255) / 256) * 256; };
    w.lut_k = 0;
    w.lut_v = al(w.lut_k + n_chunks * LQ_STREAMS * kL * 4);
    w.s0 = al(w.lut_v + n_chunks * LQ_STREAMS * kL * 4);
    w.s1 = al(w.s0 + n_heads * G * n_chunks * T * 4);
    w.rec = al(w.s1 + n_heads * G * n_chunks * T * 4);
    w.total = al(w.rec + n_chunks * 2 * n_heads * gph * (int64_t)(2 * G + G * kHd) * 4);
    return w;
}

BatchArgs to_args(const lq_chunk_batch* b, const uint32_t* lut) {
    BatchArgs a;
    a.words = b->words;
    a.chunk_base = b->chunk_base;
    a.stream_woff = b->stream_woff;
    a.blk_off = b->blk_off;
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
    return b && b->words && b->tables && b->n_chunks > 0 && b->n_heads > 0 && b->bph > 0 &&
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
    float* rec = reinterpret_cast<float*>(base + w.rec);
    int rc = lq_chunk_luts(k->tables, k->n_chunks, lut_k, s);
    if (rc) return rc;
    rc = lq_chunk_luts(v->tables, v->n_chunks, lut_v, s);
    if (rc) return rc;
    const BatchArgs ak = to_args(k, lut_k), av = to_args(v, lut_v);
    const int64_t gph = ((k->bph / kBlk) + kGB - 1) / kGB;
    const dim3 grid((unsigned)(k->n_chunks * 2 * k->n_heads * gph));
    const float qk_scale = 1.0f / sqrtf((float)kHd);
    const int64_t nq = k->n_heads * group;
#define LQ_ATTN(GG)                                                                                              \
    do {                                                                                                         \
        hipLaunchKernelGGL((k_attn_qk<GG>), grid, dim3(256), 0, s, ak, d_q, S0, S1);                             \
        hipLaunchKernelGGL((k_attn_pv<GG>), grid, dim3(256), 0, s, av, S0, S1, qk_scale, rec);       \
        hipLaunchKernelGGL((k_attn_combine<GG>), dim3((unsigned)nq), dim3(256), 0, s, rec, k->n_chunks,          \
                           k->n_heads, gph, d_q, d_tail_k, d_tail_v, t_tail, qk_scale, d_out);                   \
    } while (0)
    if (group == 1) LQ_ATTN(1);
    else if (group == 2) LQ_ATTN(2);
    else if (group == 4) LQ_ATTN(4);
    else LQ_ATTN(8);
#undef LQ_ATTN
    return launch_status();
}

}  // extern "C"
