// Fixed-rate E8 storage kernels for gfx950 (b = 3, 4, 5 bits per dimension):
// pack / unpack + dequant and the single-pass repr / fallback merge.
//
// Layout (reference core/compact_storage.py:87-154): one big-endian b-byte
// word per vector, [coset(1) | c0..c6 (b each) | c7 >> 1 (b-1)], coordinates
// biased by R = 2^(b-1).  c7's low bit is recovered from the parity of
// c0 + .. + c6 (floor-mod, as unpack_e8 does).
#include "lq_device.h"

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

__global__ void k_merge_count(const uint8_t* __restrict__ mask, int64_t total, int64_t* __restrict__ tile_cnt) {
    __shared__ int part[4];
    const int64_t t0 = (int64_t)blockIdx.x * kTile;
    int c = 0;
    for (int i = threadIdx.x; i < kTile; i += 256) {
        int64_t b = t0 + i;
        c += (b < total && mask[b]) ? 1 : 0;
    }
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) tile_cnt[blockIdx.x] = part[0] + part[1] + part[2] + part[3];
}

__global__ void k_merge_scan(int64_t n_tiles, int64_t* __restrict__ tile_cnt) {   // in place, exclusive
    __shared__ int64_t part[256];
    const int tid = threadIdx.x;
    const int64_t per = (n_tiles + 255) / 256;
    const int64_t a = tid * per, b = a + per < n_tiles ? a + per : n_tiles;
    int64_t s = 0;
    for (int64_t i = a; i < b; i++) s += tile_cnt[i];
    part[tid] = s;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        int64_t v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    int64_t run = tid ? part[tid - 1] : 0;
    for (int64_t i = a; i < b; i++) { int64_t c = tile_cnt[i]; tile_cnt[i] = run; run += c; }
}

// One tile of kTile blocks per workgroup; ranks from the tile offset plus
// wave ballots, then either unpack the packed word or copy the fp16 fallback.
__global__ __launch_bounds__(256) void k_merge(const uint8_t* __restrict__ packed, int bits,
                                               const uint16_t* __restrict__ fallback, const uint8_t* __restrict__ mask,
                                               const float* __restrict__ scales, int64_t total, int64_t bph,
                                               int64_t n_packed, int64_t n_fallback,
                                               const int64_t* __restrict__ tile_off, uint16_t* __restrict__ out) {
    __shared__ int wcnt[kTile / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t t0 = (int64_t)blockIdx.x * kTile;
    int m[4];
    for (int r = 0; r < 4; r++) {
        int64_t b = t0 + r * 256 + tid;
        m[r] = (b < total && mask[b]) ? 1 : 0;
        unsigned long long bal = __ballot(m[r]);
        if (lane == 0) wcnt[r * 4 + wave] = __popcll(bal);
    }
    __syncthreads();
    for (int r = 0; r < 4; r++) {
        int64_t b = t0 + r * 256 + tid;
        unsigned long long bal = __ballot(m[r]);
        if (b >= total) continue;
        int before = 0;
        for (int k = 0; k < r * 4 + wave; k++) before += wcnt[k];
        int64_t rr = tile_off[blockIdx.x] + before + __popcll(bal & ((1ull << lane) - 1ull));
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
    return ((total_blocks + kTile - 1) / kTile + 1) * 8;
}

int lq_fused_merge(const uint8_t* d_packed, int64_t n_packed, int bits, const uint16_t* d_fallback, int64_t n_fallback,
                   const uint8_t* d_mask, const float* d_scales, int64_t total_blocks, int64_t bph, void* d_work,
                   uint16_t* d_out, hipStream_t s) {
    if (bits < 3 || bits > 5 || total_blocks < 0 || bph <= 0 || n_packed < 0 || n_fallback < 0) return LQ_ERR_ARG;
    if (total_blocks == 0) return LQ_OK;
    const int64_t tiles = (total_blocks + kTile - 1) / kTile;
    int64_t* off = reinterpret_cast<int64_t*>(d_work);
    hipLaunchKernelGGL(k_merge_count, dim3((unsigned)tiles), dim3(256), 0, s, d_mask, total_blocks, off);
    hipLaunchKernelGGL(k_merge_scan, dim3(1), dim3(256), 0, s, tiles, off);
    hipLaunchKernelGGL(k_merge, dim3((unsigned)tiles), dim3(256), 0, s, d_packed, bits, d_fallback, d_mask, d_scales,
                       total_blocks, bph, n_packed, n_fallback, off, d_out);
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
