// Per-head scales of a chunk batch, shared by the codec (e8.hip) and the
// fixed-rate path (compact.hip), so both compute the same sigma^2, scales and
// fast-division flags: the partial sums of x^2 per (head, part), the scale
// formula of _compress_tensor and the exhaustive fast-division check.
#pragma once

#include "lq_device.h"

namespace lq {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Sum of the 8 squares of one fp16 / bf16 vector in fp32 (each square is exact
// in fp32): v_dot2 on fp16 pairs, an FMA chain for bf16.
__device__ __forceinline__ float sq_vec16(const u32x4 w, bool f16) {
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    float a = 0.f;
    if (f16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const half2_t h = __builtin_bit_cast(half2_t, d[i]);
            a = __builtin_amdgcn_fdot2(h, h, a, false);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float lo = __uint_as_float(d[i] << 16), hi = __uint_as_float(d[i] & 0xffff0000u);
            a = __builtin_fmaf(lo, lo, a);
            a = __builtin_fmaf(hi, hi, a);
        }
    }
    return a;
}

// Partial sums of x^2 per head in double: grid (heads, parts).  ROT: of the
// forward-rotated rows w = RHT(x) instead (sign row = the head, lpr lanes per
// row; the parts split on row boundaries), summed exactly like an fp32 input
// holding w, so the scales equal those of the materialised rotation.
// One (head h, part p) on a 256-thread workgroup; red: 256 doubles of LDS.
// LPR > 0: lpr as a compile-time constant (straight-line butterfly stages).
template <bool ROT, int LPR = 0>
__device__ __forceinline__ void head_sumsq_part(const void* __restrict__ x, int dtype, int64_t vec_per_head,
                                                int parts, int64_t h, int p, double* __restrict__ work, double* red,
                                                const float* __restrict__ signs, int lpr, float rdiv) {
    int64_t per = (vec_per_head + parts - 1) / parts;
    if (ROT) per = (per + lpr - 1) / lpr * lpr;
    int64_t v0 = (int64_t)p * per, v1 = v0 + per < vec_per_head ? v0 + per : vec_per_head;
    // Per vector: the 8 squares (exact in fp32 for fp16 / bf16 inputs) summed
    // in fp32, then accumulated in fp64 (four accumulators).
    double acc4[4] = {0.0, 0.0, 0.0, 0.0};
    const int64_t bd = blockDim.x;
    int64_t v = v0 + threadIdx.x;
    if (ROT) {
        // rows are whole within [v0, v1) and lpr divides the block size, so the
        // lanes of a row enter and leave the loop together
        const int lw = LPR > 0 ? LPR : lpr;
        const int part = (int)(threadIdx.x % lw);
        const float rrcp = 1.0f / rdiv;
        float sg[8];
        load_signs8(signs + h * (8 * (int64_t)lw) + 8 * part, sg);
        if (dtype == LQ_F16) {   // no range test: zero's sign does not change its square
            for (; v < v1; v += bd) {
                float xv[8];
                load8(x, LQ_F16, h * vec_per_head + v, xv);
                rht_lanes<true>(xv, sg, part, lw, rdiv, rrcp, false);
#pragma unroll
                for (int i = 0; i < 8; i++) acc4[0] += (double)xv[i] * (double)xv[i];
            }
        } else {
            for (; v < v1; v += bd) {
                float xv[8];
                load8(x, dtype, h * vec_per_head + v, xv);
                rht_lanes(xv, sg, part, lw, rdiv, rrcp, false);
#pragma unroll
                for (int i = 0; i < 8; i++) acc4[0] += (double)xv[i] * (double)xv[i];
            }
        }
    } else if (dtype == LQ_F32) {   // fp32 squares are not exact: keep every product in fp64
        for (; v < v1; v += bd) {
            float xv[8];
            load8(x, dtype, h * vec_per_head + v, xv);
#pragma unroll
            for (int i = 0; i < 8; i++) acc4[0] += (double)xv[i] * (double)xv[i];
        }
    } else {
        // eight streaming (nontemporal) 16-byte loads in flight per thread:
        // the input is read once here and once by the quantizer, too far
        // apart for the caches to keep it
        const bool f16 = dtype == LQ_F16;
        const u32x4* src = reinterpret_cast<const u32x4*>(x) + h * vec_per_head;
        for (; v + 7 * bd < v1; v += 8 * bd) {
            u32x4 w[8];
#pragma unroll
            for (int u = 0; u < 8; u++) w[u] = __builtin_nontemporal_load(src + v + u * bd);
#pragma unroll
            for (int u = 0; u < 8; u++) acc4[u & 3] += (double)sq_vec16(w[u], f16);
        }
        for (; v < v1; v += bd) acc4[0] += (double)sq_vec16(__builtin_nontemporal_load(src + v), f16);
    }
    const double acc = (acc4[0] + acc4[1]) + (acc4[2] + acc4[3]);
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) work[h * parts + p] = red[0];
}

// Exhaustive check that the three-op division equals IEEE division for every
// fp16 significand M in [1, 2047] (every fp16 value is M * 2^E, and both forms
// are invariant under that power of two), by the whole workgroup; bad: an LDS
// word.  Returns 1 (fast division exact) or 0, in every thread.
__device__ __forceinline__ int fastdiv_flag(float s, int* bad) {
    if (threadIdx.x == 0) *bad = 0;
    __syncthreads();
    const float r = 1.0f / s;
    int mine = 0;
    for (int m = 1 + (int)threadIdx.x; m < 2048; m += (int)blockDim.x) {
        const float xv = (float)m;
        const float qi = xv / s;
        const float qf = div_scaled(xv, s, r, true);
        mine |= __float_as_uint(qi) != __float_as_uint(qf);
    }
    if (mine) atomicOr(bad, 1);
    __syncthreads();
    return *bad ? 0 : 1;
}

// The fast-division word of scale s: 0, or the bits of r = RN(1 / s) (a
// positive float, so never 0) when fastdiv_flag passes.
__device__ __forceinline__ int32_t fastdiv_word(float s, int* bad) {
    const int f = fastdiv_flag(s, bad);
    return f ? __float_as_int(1.0f / s) : 0;
}

// sumsq parts per head (about 4096 workgroups in all, at most one per 512 vectors)
inline int head_parts(int64_t H, int64_t bph) {
    const int64_t want = (4096 + H - 1) / H, cap = bph / 512 > 1 ? bph / 512 : 1;
    return (int)(want < cap ? want : cap);
}

// sigma^2 (one rounding of the fp64 mean) and the scale of a head at b bits
// per dimension (llm/compressed_kv_cache.py:189-196): sqrt(RN32(f32(2 pi e) *
// sigma^2) * 4^-b), 1 where sigma^2 < f32(1e-12).
__device__ __forceinline__ float head_scale(double sum, int64_t elems, int b, float* s2_out) {
    const float s2 = (float)(sum / (double)elems);
    const float pw = ldexpf(1.0f, -2 * b);            // 4.0 ** -b, exact
    const float tv = (0x1.114580p+4f * s2) * pw;      // RN32(f32(2*pi*e) * s2) * 4^-b
    float s = sqrtf(tv);
    if (s2 < 0x1.197998p-40f) s = 1.0f;               // sigma2 < f32(1e-12)
    *s2_out = s2;
    return s;
}

}  // namespace lq

