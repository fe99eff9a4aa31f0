// Coarse / fine escape for streams whose alphabet exceeds L = 1024 symbols.
//
// The reference's table normalisation (core/gpu_ans.py:73-84) never ends for
// such a stream: it cannot bring the sum of max(f, 1) over more than L
// symbols down to L.  This build codes them instead (a build-defined format;
// the reference has none): for each coordinate j of a chunk, the least shift
// k_j >= 0 is chosen such that both cosets' streams of coordinate j span at
// most L symbols once shifted, i.e. (max >> k) - (min >> k) + 5 <= L.  The
// stream then carries the coarse symbols s >> k_j (floor division) through
// the unchanged table / rANS path, and the k_j low bits s & (2^k_j - 1) of
// every vector are stored raw: coordinate j of a chunk owns nblk * 16 * k_j
// words, vector v's bits at bit v * k_j, least significant bit first (a block
// of 512 vectors fills exactly 16 * k_j words).  k_j = 0 for every coordinate
// of a chunk whose alphabets fit, which then stays the reference's format.
#include <climits>

#include "lq_device.h"

using namespace lq;

namespace {

inline int launch_status() { return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_LAUNCH; }

constexpr int kMaxShift = LQ_ESC_MAX_SHIFT;   // int16 symbols span < 2^16: k = 7 leaves at most 512 + 5 coarse symbols

__device__ __forceinline__ int64_t span_after(int mn, int mx, int k) {
    return (int64_t)(mx >> k) - (int64_t)(mn >> k) + 5;
}

// One wave per chunk; lane j < 8 plans coordinate j: esc_k[chunk * 8 + j] and
// the coarse (min, max) of streams (0, j) and (1, j) (absent streams keep
// their empty marker).  A coordinate no shift can fit sets LQ_ST_ALPHABET.
__global__ __launch_bounds__(64) void k_chunk_esc_plan(const int32_t* __restrict__ minmax, int32_t* __restrict__ esc_k,
                                                       int32_t* __restrict__ minmax_c, int32_t* __restrict__ status) {
    const int64_t chunk = blockIdx.x;
    const int j = threadIdx.x;
    if (j >= 8) return;
    int mn[2], mx[2];
    bool present[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int64_t sid = chunk * LQ_STREAMS + c * 8 + j;
        mn[c] = minmax[2 * sid];
        mx[c] = minmax[2 * sid + 1];
        present[c] = mx[c] != INT_MIN;
    }
    int k = 0;
    while (k <= kMaxShift &&
           ((present[0] && span_after(mn[0], mx[0], k) > kL) || (present[1] && span_after(mn[1], mx[1], k) > kL)))
        k++;
    if (k > kMaxShift) {
        atomicOr(status + chunk, LQ_ST_ALPHABET);
        k = 0;
    }
    esc_k[chunk * 8 + j] = k;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int64_t sid = chunk * LQ_STREAMS + c * 8 + j;
        minmax_c[2 * sid] = present[c] ? (mn[c] >> k) : mn[c];
        minmax_c[2 * sid + 1] = present[c] ? (mx[c] >> k) : mx[c];
    }
}

// One workgroup per (block, chunk), one thread per vector of the block: the
// int16 staging of every escaped coordinate becomes its coarse symbols in
// place, and each vector's low bits wait in LDS (one byte per vector and
// coordinate, k <= 7); then every thread assembles whole fine words -- word t
// of coordinate j holds bits 32 t .. 32 t + 31 of the coordinate's bit string,
// vector v's k bits at bit v k -- from the vectors those bits come from, and
// stores them (no LDS atomics: vectors sharing a word would serialise on
// its address).  Vectors past the chunk's end contribute zero bits.
__global__ __launch_bounds__(kBlk) void k_chunk_esc_split(int16_t* __restrict__ sym, const uint8_t* __restrict__ coset_bits,
                                                          const uint32_t* __restrict__ blk_n1, int64_t nblk, int64_t V,
                                                          const int32_t* __restrict__ esc_k,
                                                          const int64_t* __restrict__ fine_off,
                                                          uint32_t* __restrict__ fine) {
    __shared__ uint8_t fv[8][kBlk];
    __shared__ uint32_t bm[kBlk / 32];
    const int64_t chunk = blockIdx.y, g = blockIdx.x;
    const int tid = threadIdx.x;
    int kk[8];
    int any = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        kk[j] = esc_k[chunk * 8 + j];
        any |= kk[j];
    }
    if (!any) return;   // chunk-uniform
    if (tid < kBlk / 32) bm[tid] = reinterpret_cast<const uint32_t*>(coset_bits + (chunk * nblk + g) * (kBlk / 8))[tid];
    __syncthreads();
    const int valid = (int)(V - g * kBlk < kBlk ? V - g * kBlk : kBlk);
    if (tid < valid) {
        const int n1 = (int)blk_n1[chunk * nblk + g];
        const int n0 = valid - n1;
        const int w = tid >> 5;
        int below = 0;   // coset-1 vectors of the block before this one
        for (int i = 0; i < w; i++) below += __builtin_popcount(bm[i]);
        below += __builtin_popcount(bm[w] & ((1u << (tid & 31)) - 1u));
        const int c = (bm[w] >> (tid & 31)) & 1;
        const int r = c ? below : tid - below;
        int16_t* blk = sym + (chunk * nblk + g) * (int64_t)kSymStride;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int k = kk[j];
            if (k == 0) continue;
            int16_t* p = blk + sym_pos(c, j, r, n0);
            const int s = *p;
            *p = (int16_t)(s >> k);
            fv[j][tid] = (uint8_t)((uint32_t)s & ((1u << k) - 1u));
        }
    }
    __syncthreads();
    // the block's fine words, coordinates in order: 16 k_j words each
    int nw = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) nw += 16 * kk[j];
    for (int t = tid; t < nw; t += kBlk) {
        int j = 0, tj = t;
        while (tj >= 16 * kk[j]) { tj -= 16 * kk[j]; j++; }   // kk[j] > 0 where the loop stops
        const int k = kk[j];
        const int b0 = 32 * tj;
        const int v0 = b0 / k;
        const int v1 = (b0 + 31) / k < valid - 1 ? (b0 + 31) / k : valid - 1;
        uint32_t word = 0u;
        for (int v = v0; v <= v1; v++) {
            const int sh = v * k - b0;   // position of vector v's lowest bit in the word
            const uint32_t f = fv[j][v];
            word |= sh >= 0 ? f << sh : f >> -sh;
        }
        fine[fine_off[chunk * 8 + j] + g * 16 * k + tj] = word;
    }
}

}  // namespace

extern "C" {

int lq_chunk_escape_plan(const int32_t* d_minmax, int64_t n_chunks, int32_t* d_esc_k, int32_t* d_minmax_coarse,
                         int32_t* d_status, hipStream_t s) {
    if (n_chunks <= 0 || !d_minmax || !d_esc_k || !d_minmax_coarse || !d_status) return LQ_ERR_ARG;
    hipLaunchKernelGGL(k_chunk_esc_plan, dim3((unsigned)n_chunks), dim3(64), 0, s, d_minmax, d_esc_k, d_minmax_coarse,
                       d_status);
    return launch_status();
}

int lq_chunk_escape_split(int16_t* d_sym, const uint8_t* d_coset_bits, const uint32_t* d_blk_n1, int64_t n_chunks,
                          int64_t n_vectors, const int32_t* d_esc_k, const int64_t* d_fine_off, uint32_t* d_fine,
                          hipStream_t s) {
    if (n_chunks <= 0 || n_vectors <= 0 || !d_sym || !d_coset_bits || !d_blk_n1 || !d_esc_k || !d_fine_off || !d_fine)
        return LQ_ERR_ARG;
    const int64_t nblk = (n_vectors + kBlk - 1) / kBlk;
    hipLaunchKernelGGL(k_chunk_esc_split, dim3((unsigned)nblk, (unsigned)n_chunks), dim3(kBlk), 0, s, d_sym,
                       d_coset_bits, d_blk_n1, nblk, n_vectors, d_esc_k, d_fine_off, d_fine);
    return launch_status();
}

}  // extern "C"
