// Element-wise helpers behind the reference's Python API (gfx950):
// E8 validation, fixed-rate unpack to lattice points, symbol -> table index
// mapping for rans_encode, coset bit packing, and the randomized Hadamard
// transform of core/pipeline.py.
#include <cmath>

#include "lq_device.h"

using namespace lq;

namespace {

inline int launch_status() { return hipGetLastError() == hipSuccess ? LQ_OK : LQ_ERR_LAUNCH; }

// validate_e8 + check_representable (core/compact_storage.py:39-80, 235-249).
// flags: LQ_V_VALID | LQ_V_HALF | LQ_V_INRANGE (in range for `bits`, when 3 <= bits <= 5).
__global__ void k_validate(const float* __restrict__ q, int64_t n, float atol, int bits, int32_t* __restrict__ flags) {
    int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n) return;
    float p[8];
    load8(q, LQ_F32, v, p);
    float ri = 0.f, rh = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        ri = fmaxf(ri, fabsf(p[i] - rintf(p[i])));
        const float h = p[i] - 0.5f;
        rh = fmaxf(rh, fabsf(h - rintf(h)));
    }
    // a NaN residual compares false in both checks, as torch's max(...) < atol does
    const bool is_int = ri < atol, is_half = rh < atol;
    int64_t sum = 0;
    bool in_range = true;
    const int64_t R = bits >= 3 && bits <= 5 ? (1ll << (bits - 1)) : 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float t = rintf(is_half ? p[i] - 0.5f : p[i]);
        // torch's .long() of a float outside int64 is undefined; such points are invalid anyway
        const int64_t c = (fabsf(t) < 9.0e18f) ? (int64_t)t : 0;
        sum += c;
        in_range = in_range && c >= -R && c <= R - 1;
    }
    const bool valid = (is_int || is_half) && ((sum & 1) == 0);
    int32_t f = (valid ? LQ_V_VALID : 0) | (is_half ? LQ_V_HALF : 0);
    if (R && valid && in_range) f |= LQ_V_INRANGE;
    flags[v] = f;
}

__device__ __forceinline__ uint64_t load_be(const uint8_t* p, int bits) {
    uint64_t w = 0;
    for (int b = 0; b < bits; b++) w = (w << 8) | p[b];
    return w;
}

// unpack_e8 (core/compact_storage.py:157-222) to fp32 lattice points.
__global__ void k_unpack_f32(const uint8_t* __restrict__ packed, int bits, int64_t n, float* __restrict__ q) {
    int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n) return;
    uint64_t w = bits == 4 ? (uint64_t)__builtin_bswap32(reinterpret_cast<const uint32_t*>(packed)[v])
                           : load_be(packed + v * bits, bits);
    const int R = 1 << (bits - 1);
    const uint64_t cm = (1ull << bits) - 1ull, um = (1ull << (bits - 1)) - 1ull;
    const int c7u = (int)(w & um);
    w >>= (bits - 1);
    int c[7], ps = 0;
#pragma unroll
    for (int i = 6; i >= 0; i--) { c[i] = (int)(w & cm) - R; w >>= bits; }
    const float off = (w & 1ull) ? 0.5f : 0.f;
#pragma unroll
    for (int i = 0; i < 7; i++) ps += c[i];
    float o[8];
#pragma unroll
    for (int i = 0; i < 7; i++) o[i] = (float)c[i] + off;
    o[7] = (float)(c7u * 2 + (ps & 1) - R) + off;
    store8(q, LQ_F32, v, o);
}

// Symbol value -> table index as rans_encode resolves it (core/gpu_ans.py:110-119):
// the index of an equal alphabet entry (the last one, as the dict keeps), else
// the first entry at minimal |alphabet[i] - s|.  contiguous != 0: the alphabet is
// lo, lo+1, .., lo+n-1, where that reduces to clamp(s - lo, 0, n - 1).
__global__ __launch_bounds__(256) void k_symbol_index(const int64_t* __restrict__ sym, int64_t n,
                                                      const int64_t* __restrict__ alph, int n_alph, int contiguous,
                                                      int32_t* __restrict__ idx) {
    __shared__ int64_t a[LQ_L];
    if (!contiguous)
        for (int i = threadIdx.x; i < n_alph; i += blockDim.x) a[i] = alph[i];
    __syncthreads();
    const int64_t lo = alph[0];
    for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < n; v += (int64_t)gridDim.x * blockDim.x) {
        const int64_t s = sym[v];
        int r;
        if (contiguous) {
            const int64_t d = s - lo;
            r = d < 0 ? 0 : (d >= n_alph ? n_alph - 1 : (int)d);
        } else {
            int exact = -1, best = 0;
            uint64_t bd = ~0ull;
            for (int i = 0; i < n_alph; i++) {
                const int64_t t = a[i];
                if (t == s) exact = i;
                const uint64_t dd = t > s ? (uint64_t)(t - s) : (uint64_t)(s - t);
                if (dd < bd) { bd = dd; best = i; }
            }
            r = exact >= 0 ? exact : best;
        }
        idx[v] = r;
    }
}

// pack_coset_bits (llm/compressed_kv_cache.py:46-54): bit i of the output is coset[i] & 1,
// bytes LSB-first.  One thread per output byte.
__global__ void k_pack_bits(const uint8_t* __restrict__ coset, int64_t n, uint8_t* __restrict__ out) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= (n + 7) / 8) return;
    uint32_t b = 0;
    for (int k = 0; k < 8; k++) {
        const int64_t i = 8 * j + k;
        if (i < n) b |= (uint32_t)(coset[i] & 1u) << k;
    }
    out[j] = (uint8_t)b;
}

// unpack_coset_bits (llm/compressed_kv_cache.py:57-63).
__global__ void k_unpack_bits(const uint8_t* __restrict__ packed, int64_t n, uint8_t* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = (uint8_t)((packed[i >> 3] >> (i & 7)) & 1u);
}

// Randomized Hadamard transform of d-dim rows (rht_lanes: core/pipeline.py:49-118,
// llm/perplexity_eval.py:35-61), d/8 lanes per row, 8 consecutive elements per
// lane.  Row r uses sign row (r / rows_per_sign) % n_sign.
template <int IN_DT, int OUT_DT>
__global__ __launch_bounds__(256) void k_rht(const void* __restrict__ x, int64_t n_rows, int d, const float* __restrict__ signs,
                                             int64_t rows_per_sign, int n_sign, float div, int inverse,
                                             void* __restrict__ out) {
    const int lpr = d >> 3;   // lanes per row (1..64, power of two)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t row = t / lpr;
    const int part = (int)(t % lpr);
    const bool live = row < n_rows;
    const int64_t rr = live ? row : 0;
    const int64_t v = rr * lpr + part;   // 8-element vector index
    float y[8], s[8];
    load8(x, IN_DT, v, y);
    load_signs8(signs + ((rr / rows_per_sign) % n_sign) * (int64_t)d + 8 * part, s);
    // lanes of one row are consecutive and lpr divides 64, so rows never straddle a wave
    rht_lanes(y, s, part, lpr, div, 1.0f / div, inverse != 0);
    if (live) store8(out, OUT_DT, v, y);
}

}  // namespace

extern "C" {

int lq_e8_validate(const float* d_q, int64_t n, float atol, int bits, int32_t* d_flags, hipStream_t s) {
    if (n < 0) return LQ_ERR_ARG;
    if (n == 0) return LQ_OK;
    hipLaunchKernelGGL(k_validate, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_q, n, atol, bits, d_flags);
    return launch_status();
}

int lq_unpack_e8(const uint8_t* d_packed, int bits, int64_t n, float* d_q, hipStream_t s) {
    if (bits < 3 || bits > 5 || n < 0) return LQ_ERR_ARG;
    if (n == 0) return LQ_OK;
    hipLaunchKernelGGL(k_unpack_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_packed, bits, n, d_q);
    return launch_status();
}

int lq_symbol_index(const int64_t* d_sym, int64_t n, const int64_t* d_alphabet, int32_t n_alphabet, int contiguous,
                    int32_t* d_idx, hipStream_t s) {
    if (n < 0 || n_alphabet <= 0 || n_alphabet > LQ_L) return LQ_ERR_ARG;
    if (n == 0) return LQ_OK;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(k_symbol_index, dim3((unsigned)blocks), dim3(256), 0, s, d_sym, n, d_alphabet, n_alphabet,
                       contiguous, d_idx);
    return launch_status();
}

int lq_pack_coset_bits(const uint8_t* d_coset, int64_t n, uint8_t* d_out, hipStream_t s) {
    if (n < 0) return LQ_ERR_ARG;
    if (n == 0) return LQ_OK;
    const int64_t nb = (n + 7) / 8;
    hipLaunchKernelGGL(k_pack_bits, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, d_coset, n, d_out);
    return launch_status();
}

int lq_unpack_coset_bits(const uint8_t* d_packed, int64_t n, uint8_t* d_out, hipStream_t s) {
    if (n < 0) return LQ_ERR_ARG;
    if (n == 0) return LQ_OK;
    hipLaunchKernelGGL(k_unpack_bits, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, d_packed, n, d_out);
    return launch_status();
}

int lq_rht(const void* d_x, int in_dtype, int64_t n_rows, int d, const float* d_signs, int64_t rows_per_sign,
           int n_sign, int inverse, void* d_out, int out_dtype, hipStream_t s) {
    if (n_rows < 0 || d < 8 || d > 512 || (d & (d - 1)) || rows_per_sign <= 0 || n_sign <= 0) return LQ_ERR_ARG;
    if (in_dtype < 0 || in_dtype > 2 || out_dtype < 0 || out_dtype > 2) return LQ_ERR_ARG;
    if (n_rows == 0) return LQ_OK;
    const float div = (float)sqrt((double)d);   // f32(np.sqrt(d)), the divisor torch applies
    const int64_t threads = n_rows * (d / 8);
    const dim3 grid((unsigned)((threads + 255) / 256));
#define LQ_RHT(I, O) \
    hipLaunchKernelGGL((k_rht<I, O>), grid, dim3(256), 0, s, d_x, n_rows, d, d_signs, rows_per_sign, n_sign, div, inverse, d_out)
    if (in_dtype == LQ_F16) { if (out_dtype == LQ_F32) LQ_RHT(LQ_F16, LQ_F32); else if (out_dtype == LQ_F16) LQ_RHT(LQ_F16, LQ_F16); else LQ_RHT(LQ_F16, LQ_BF16); }
    else if (in_dtype == LQ_BF16) { if (out_dtype == LQ_F32) LQ_RHT(LQ_BF16, LQ_F32); else if (out_dtype == LQ_F16) LQ_RHT(LQ_BF16, LQ_F16); else LQ_RHT(LQ_BF16, LQ_BF16); }
    else { if (out_dtype == LQ_F32) LQ_RHT(LQ_F32, LQ_F32); else if (out_dtype == LQ_F16) LQ_RHT(LQ_F32, LQ_F16); else LQ_RHT(LQ_F32, LQ_BF16); }
#undef LQ_RHT
    return launch_status();
}

}  // extern "C"
