// Device helpers shared by the LatticeQuant gfx950 kernels.
//
// All fp32 arithmetic that decides a lattice point is written so that it
// rounds exactly where the reference's torch ops round (the library is built
// with -ffp-contract=off; FMAs appear only where written explicitly).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

#include "latticequant_amd.h"

namespace lq {

constexpr int kL = LQ_L;
constexpr int kBlk = LQ_BLK;
constexpr int kCapW = (10 * LQ_BLK + 31) / 32;   // scratch words per (stream, block) task
constexpr int kSymStride = LQ_SYM_STRIDE;        // bytes of int8 symbols per block

// Symbols of one block: the coset-0 region then the coset-1 region, each
// holding its 8 equal-length coordinate columns interleaved in 16-byte units
// (chunk k of column i at (8 k + i) * 16), so the 8 lanes that walk the 8
// columns of a (block, coset) together read one full 128-byte line per step.
// Byte offset of rank r of column i of coset c, given the block's coset-0 count.
__device__ __forceinline__ int sym_region(int c, int n0) { return c ? 128 * ((n0 + 15) >> 4) : 0; }
__device__ __forceinline__ int sym_pos(int c, int i, int r, int n0) {
    return sym_region(c, n0) + ((((r >> 4) << 3) + i) << 4) + (r & 15);
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4_t gconst_u32x4;

// 16-byte load through a global (address space 1) pointer: a global_load, not
// a flat load, so it does not hold up waits on LDS results.
__device__ __forceinline__ uint4 gload16(uintptr_t a) {
    u32x4_t v = *reinterpret_cast<gconst_u32x4*>(a);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 symbols of one column chunk (int8: one 16-byte load, int16: two).
template <typename SymT>
struct Chunk16 {
    uint4 a, b;
    __device__ __forceinline__ int get(int i) const {
        if constexpr (sizeof(SymT) == 1) {
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
            return (int)(int8_t)(w[i >> 2] >> ((i & 3) * 8));
        } else {
            const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            return (int)(int16_t)(w[i >> 1] >> ((i & 1) * 16));
        }
    }
};

template <typename SymT>
__device__ __forceinline__ Chunk16<SymT> gload_chunk(const SymT* p) {
    Chunk16<SymT> c;
    const uintptr_t a = (uintptr_t)p;
    c.a = gload16(a);
    if constexpr (sizeof(SymT) == 2) c.b = gload16(a + 16);
    else c.b = make_uint4(0, 0, 0, 0);
    return c;
}

// torch.arange(8, dtype=f32) * 1e-7  ==  RN32(i * f32(1e-7))   (core/e8_quantizer.py:42-44)
__host__ __device__ __forceinline__ float tiebreak(int i) {
    constexpr float tb[8] = {0.0f,           0x1.ad7f2ap-24f, 0x1.ad7f2ap-23f, 0x1.421f60p-22f,
                             0x1.ad7f2ap-22f, 0x1.0c6f7ap-21f, 0x1.421f60p-21f, 0x1.77cf44p-21f};
    return tb[i];
}

// ---------------------------------------------------------------- dtypes --
__device__ __forceinline__ float h2f(uint16_t u) { return __half2float(__ushort_as_half(u)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }
__device__ __forceinline__ float bf2f(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {   // round to nearest even, quiet NaN
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Load one 8-dim vector (index v) of an fp16 / bf16 / fp32 array as fp32.
__device__ __forceinline__ void load8(const void* base, int dtype, int64_t v, float x[8]) {
    if (dtype == LQ_F32) {
        const float4* p = reinterpret_cast<const float4*>(base) + 2 * v;
        float4 a = p[0], b = p[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
        uint4 r = reinterpret_cast<const uint4*>(base)[v];
        uint32_t w[4] = {r.x, r.y, r.z, r.w};
        if (dtype == LQ_F16) {   // dtype is uniform: one branch, not a select per element
#pragma unroll
            for (int i = 0; i < 4; i++) {
                x[2 * i] = h2f((uint16_t)(w[i] & 0xffffu));
                x[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                x[2 * i] = __uint_as_float(w[i] << 16);
                x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            }
        }
    }
}

__device__ __forceinline__ void store8(void* base, int dtype, int64_t v, const float y[8]) {
    if (dtype == LQ_F32) {
        float4* p = reinterpret_cast<float4*>(base) + 2 * v;
        p[0] = make_float4(y[0], y[1], y[2], y[3]);
        p[1] = make_float4(y[4], y[5], y[6], y[7]);
    } else {
        uint32_t w[4];
        for (int i = 0; i < 4; i++) {
            uint16_t lo = dtype == LQ_F16 ? f2h(y[2 * i]) : f2bf(y[2 * i]);
            uint16_t hi = dtype == LQ_F16 ? f2h(y[2 * i + 1]) : f2bf(y[2 * i + 1]);
            w[i] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        reinterpret_cast<uint4*>(base)[v] = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

__device__ __forceinline__ uint16_t f2dtype(float f, int dtype) { return dtype == LQ_F16 ? f2h(f) : f2bf(f); }

// ------------------------------------------------------------------- E8 ---

// Nearest D8 point (core/e8_quantizer.py:20-58): round half-even, and when the
// coordinate sum is odd move the coordinate with the smallest
// RN(RN(1 - 2|r|) + tiebreak_i) (first index on ties) one step away from x.
__host__ __device__ __forceinline__ void d8_round(const float x[8], float r[8]) {
    float res[8];
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = rintf(x[i]);
    float s = r[0];
#pragma unroll
    for (int i = 1; i < 8; i++) s += r[i];
    // first-index argmin of RN(RN(1 - 2|res_i|) + tiebreak_i): upd[i] says the
    // running minimum moved to i, so the argmin is the last i with upd[i]
    // (the per-lane flags stay lane masks; no index is materialised)
    float best = 0.f;
    bool upd[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        res[i] = x[i] - r[i];
        // RN(1 - 2|res|): 2|res| is exact, so one fused op rounds the same way
        const float fc = __builtin_fmaf(-2.0f, fabsf(res[i]), 1.0f);
        const float adj = i == 0 ? fc : fc + tiebreak(i);   // tiebreak(0) = 0 and fc is never -0
        upd[i] = i == 0 || adj < best;
        best = upd[i] ? adj : best;
    }
    bool sel[8];
    bool later = false;
#pragma unroll
    for (int i = 7; i >= 0; i--) {
        sel[i] = upd[i] && !later;
        later = later || upd[i];
    }
    // parity of the fp32 sum (torch: r.sum(-1) % 2): every fp32 value of
    // magnitude >= 2^24 is even, below that the int32 conversion is exact
    const bool odd = fabsf(s) < 16777216.0f && (((int32_t)s) & 1);
    if (odd) {
        float rv = res[0];
#pragma unroll
        for (int i = 1; i < 8; i++) rv = sel[i] ? res[i] : rv;
        const float sg = rv < 0.f ? -1.f : 1.f;   // sign(res), 0 -> +1
#pragma unroll
        for (int i = 0; i < 8; i++) r[i] = sel[i] ? r[i] + sg : r[i];
    }
}

// Nearest E8 point (core/e8_quantizer.py:61-83).  Returns the integer
// coordinates of the chosen coset representative (c1 itself, or c2 - 1/2) and
// the coset bit; the squared distances are summed left to right like torch's
// CPU sum over an 8-wide row.
__host__ __device__ __forceinline__ int e8_nearest(const float x[8], float ic[8]) {
    float r1[8], r2[8], y[8];
    d8_round(x, r1);
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = x[i] - 0.5f;
    d8_round(y, r2);
    float d1 = 0.f, d2 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float a = x[i] - r1[i];
        float b = x[i] - (r2[i] + 0.5f);
        float a2 = a * a, b2 = b * b;
        d1 = (i == 0) ? a2 : d1 + a2;
        d2 = (i == 0) ? b2 : d2 + b2;
    }
    bool use1 = d1 <= d2;
#pragma unroll
    for (int i = 0; i < 8; i++) ic[i] = use1 ? r1[i] : r2[i];
    return use1 ? 0 : 1;
}

// The same nearest E8 point as e8_nearest, with less arithmetic on the common
// path.  Both D8 roundings are taken as in d8_round, but their flips are not
// applied until the coset is known (one flip instead of two).  The coset
// choice d1 <= d2 is first decided from an estimate of d1 - d2 with a proven
// error bound; only when the estimate lies within that bound of zero are the
// two distances summed in the reference's order from the same halves.
//
// With e1 = x - r1 and e2 = y - r2 (y = RN(x - 1/2); both differences exact),
//   d1 = sum e1^2 + odd1 (1 - 2 |e1_j|),  d2 = sum e2^2 + odd2 (1 - 2 |e2_k|)
// (j, k the flipped coordinates).  |e2_i| = 1/2 - |e1_i| + s_i with |s_i| <= U,
// U the ulp of max(1, max |x_i|) (the rounding of y), so
// e1_i^2 - e2_i^2 = |e1_i| - 1/4 + O(1.01 U), and with f_i = RN(1 - 2 |e1_i|)
// (the flip costs d8_half computes anyway)
//   d1 - d2 ~ est = 2 - (sum f_i) / 2 + odd1 f1_j - odd2 f2_k.
// The error of est against the exact d1 - d2 (the s_i, the rounding of the
// reference's differences x - c, of the f_i and of the fp32 evaluation, <= 1.9e-6)
// plus the reference's own rounding of its sums (<= 9 * 2^-24 relative on
// d <= 4) stays below 1e-5 + 32 U; beyond that margin the sign of est is the
// sign of the reference's fp32 d1 - d2.  max |x_i| >= 2^21 (or inf / NaN
// through est) takes the exact path.
struct D8Half {
    float r[8], e[8];
    bool sel[8];   // first-index argmin of RN(RN(1 - 2|e_i|) + tiebreak_i)
    float es;      // e at that index
    float fsum;    // sum of RN(1 - 2|e_i|) (left to right), when asked for
    bool odd;      // the fp32 coordinate sum is odd
};

template <bool FSUM>
__host__ __device__ __forceinline__ void d8_half(const float x[8], D8Half& h) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        h.r[i] = rintf(x[i]);
        h.e[i] = x[i] - h.r[i];
    }
    float s = h.r[0];
#pragma unroll
    for (int i = 1; i < 8; i++) s += h.r[i];
    h.odd = fabsf(s) < 16777216.0f && (((int32_t)s) & 1);
    float best = 0.f, es = h.e[0], fs = 0.f;
    bool upd[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float fc = __builtin_fmaf(-2.0f, fabsf(h.e[i]), 1.0f);
        if (FSUM) fs = i == 0 ? fc : fs + fc;
        const float adj = i == 0 ? fc : fc + tiebreak(i);
        upd[i] = i == 0 || adj < best;
        best = upd[i] ? adj : best;
        es = upd[i] ? h.e[i] : es;
    }
    bool later = false;
#pragma unroll
    for (int i = 7; i >= 0; i--) {
        h.sel[i] = upd[i] && !later;
        later = later || upd[i];
    }
    h.es = es;
    h.fsum = fs;
}

// Reference-order coset choice (core/e8_quantizer.py:79-83) given the halves.
__host__ __device__ __forceinline__ bool e8_choose_exact(const float x[8], const D8Half& a, const D8Half& b,
                                                         float fa, float fb) {
    float d1 = 0.f, d2 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float c1 = a.r[i] + (a.sel[i] ? fa : 0.f);
        const float c2 = (b.r[i] + (b.sel[i] ? fb : 0.f)) + 0.5f;
        const float u = x[i] - c1, v = x[i] - c2;
        const float u2 = u * u, v2 = v * v;
        d1 = (i == 0) ? u2 : d1 + u2;
        d2 = (i == 0) ? v2 : d2 + v2;
    }
    return d1 <= d2;
}

// reload(float x[8]) writes x again for the rare exact path, so that x need
// not stay live through the common path.  tmax (optional) receives
// max(1, max_i |x_i|) (NaN coordinates ignored).  When tmax < T for an
// integer T, every returned coordinate lies in [-(T + 1), T + 1]: rint(x_i)
// lies in [-T, T], rint(x_i - 1/2) in [-T, T - 1], and a flip adds +-1.
// Callers can skip the range checks of their symbols then.
template <typename Reload>
__host__ __device__ __forceinline__ int e8_nearest_fast(const float x[8], float ic[8], Reload&& reload,
                                                        float* tmax = nullptr) {
    D8Half a, b;
    d8_half<true>(x, a);
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = x[i] - 0.5f;
    d8_half<false>(y, b);
    float est = __builtin_fmaf(a.fsum, -0.5f, 2.0f);
    if (a.odd) est += __builtin_fmaf(-2.0f, fabsf(a.es), 1.0f);
    if (b.odd) est -= __builtin_fmaf(-2.0f, fabsf(b.es), 1.0f);
    float t = fmaxf(fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))),
                    fmaxf(fmaxf(fabsf(x[4]), fabsf(x[5])), fmaxf(fabsf(x[6]), fabsf(x[7]))));
    t = fmaxf(t, 1.0f);
    const float p2 = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, t) & 0x7f800000u);   // 2^floor(log2 t)
    const float margin = __builtin_fmaf(32.0f * 0x1p-23f, p2, 1e-5f);   // 1e-5 + 32 ulp(t)
    // each half's flip as a float step (0 when its sum is even)
    const float fa = a.odd ? (a.es < 0.f ? -1.f : 1.f) : 0.f;
    const float fb = b.odd ? (b.es < 0.f ? -1.f : 1.f) : 0.f;
    bool use1 = est < 0.f;
    if (!(t < 2097152.0f) || !(fabsf(est) > margin)) {
        float xr[8];
        reload(xr);
        use1 = e8_choose_exact(xr, a, b, fa, fb);
    }
    if (tmax) *tmax = t;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float ca = a.r[i] + (a.sel[i] ? fa : 0.f);
        const float cb = b.r[i] + (b.sel[i] ? fb : 0.f);
        ic[i] = use1 ? ca : cb;
    }
    return use1 ? 0 : 1;
}

__host__ __device__ __forceinline__ int e8_nearest_fast(const float x[8], float ic[8]) {
    return e8_nearest_fast(x, ic, [&](float xr[8]) {
#pragma unroll
        for (int i = 0; i < 8; i++) xr[i] = x[i];
    });
}

// x / s rounded to nearest.  The three-op form (q0 = x*r, e = fma(-q0, s, x),
// q1 = fma(e, r, q0)) is used only for heads whose scale passed the exhaustive
// check of lq_scale_fastdiv; otherwise IEEE division.
__device__ __forceinline__ float div_scaled(float x, float s, float r, bool fast) {
    if (fast) {
        float q0 = x * r;
        float e = __builtin_fmaf(-q0, s, x);
        return __builtin_fmaf(e, r, q0);
    }
    return x / s;
}

// ----------------------------------------------------------------- RHT ---
//
// Randomized Hadamard transform of d-dim rows (core/pipeline.py:49-118,
// llm/perplexity_eval.py:35-61): forward w = FWHT(x * s) / sqrt(d), inverse
// v = FWHT(w) / sqrt(d) * s, in fp32.  Each butterfly stage h = 1, 2, .., d/2
// replaces (a, b) = (y[i], y[i + h]) by (a + b, a - b) as the reference loop
// does, so the fp32 result is the reference's bit for bit.  A row lies in
// lpr = d / 8 consecutive lanes (lpr divides 64), 8 consecutive elements per
// lane: stages h < 8 run in registers, h >= 8 across lanes (partner lane ^ h/8).
// Every lane of a row must execute this together.  div = f32(sqrt(d)).
//
// Partner lanes l ^ 1 .. l ^ 16 are read with one ds_swizzle each (bitmask
// mode, within 32 lanes), which issues on the LDS pipe and leaves the VALU to
// the arithmetic (these kernels are VALU-bound); the butterfly is then one
// FMA, fma(y, +-1, partner) = RN(partner +- y): the lower lane of a pair gets
// a + b, the upper a - b, bit for bit as the add / subtract.  Rows of 64
// lanes (head_dim 512) read partner l ^ 32 with a shuffle.
template <int HL>
__device__ __forceinline__ float lane_xor(float v) {
    const int i = __builtin_bit_cast(int, v);
    int r;
    if constexpr (HL <= 16) {
        // ds_swizzle in bitmask mode (offset bit 15 clear): lane (l & 0x1f) ^ HL
        // of its 32-lane half, on the LDS pipe, not the VALU
        r = __builtin_amdgcn_ds_swizzle(i, (HL << 10) | 0x1f);
    } else {
        return __shfl_xor(v, HL, 64);
    }
    return __builtin_bit_cast(float, r);
}

template <int HL>
__device__ __forceinline__ void fwht_cross_t(float y[8], int part) {
    const float sgn = (part & HL) ? -1.0f : 1.0f;   // upper lane of the pair: partner - own
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = __builtin_fmaf(y[i], sgn, lane_xor<HL>(y[i]));
}

// One butterfly stage across lanes: partner lane ^ hl (stage h = 8 hl).
__device__ __forceinline__ void fwht_cross(float y[8], int part, int hl) {
    switch (hl) {
        case 1: fwht_cross_t<1>(y, part); break;
        case 2: fwht_cross_t<2>(y, part); break;
        case 4: fwht_cross_t<4>(y, part); break;
        case 8: fwht_cross_t<8>(y, part); break;
        case 16: fwht_cross_t<16>(y, part); break;
        default: fwht_cross_t<32>(y, part); break;
    }
}

// Butterfly stages h = 1 .. 4 nl of rows spread over nl lanes: h < 8 in
// registers, then across lanes.
__device__ __forceinline__ void fwht_stages(float y[8], int part, int nl) {
#pragma unroll
    for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (i & h) continue;
            const float a = y[i], b = y[i + h];
            y[i] = a + b;
            y[i + h] = a - b;
        }
    }
    if (nl > 1) fwht_cross_t<1>(y, part);
    if (nl > 2) fwht_cross_t<2>(y, part);
    if (nl > 4) fwht_cross_t<4>(y, part);
    if (nl > 8) fwht_cross_t<8>(y, part);
    if (nl > 16) fwht_cross_t<16>(y, part);
    if (nl > 32) fwht_cross_t<32>(y, part);
}

// y / d as IEEE fp32 division rounds it, for the rotation's divisor
// d = f32(sqrt(D)), D a power of two in [8, 512], in three operations given
// r = RN(1 / d): q0 = RN(y r), the residual e = y - q0 d (exact, one FMA),
// RN(q0 + e r).  Each such d is a power of two or 2^k f32(sqrt 2), and for
// those divisors the three operations give RN(y / d) for every fp32
// significand (checked exhaustively by tests/host/div_sqrt_check.cpp), hence
// for every y whose residual stays exact: |y| >= 2^-100 suffices.  Zeros
// (whose sign the FMA form loses), tiny, infinite and NaN y take the IEEE
// division.
__host__ __device__ __forceinline__ float div_sqrt_dim(float y, float d, float r) {
    const float q0 = y * r;
    const float e = __builtin_fmaf(-q0, d, y);
    float q = __builtin_fmaf(e, r, q0);
    if (!(__builtin_fabsf(y) >= 0x1p-100f && __builtin_fabsf(y) <= 0x1.fffffep127f)) q = y / d;
    return q;
}

// x / s as IEEE fp32 division rounds it, in five operations given
// r = RN(1 / s), for |x| and s in [2^-60, 2^60] (every intermediate is then a
// normal number and each remainder x - q s is computed exactly): q0 = RN(x r)
// lies within 1.5 ulp of x / s, one correction q1 = RN(q0 + RN(x - q0 s) r)
// within one ulp, and a second correction of a quotient within one ulp with r
// within half an ulp of 1 / s is correctly rounded (Markstein 1990, IBM J. Res.
// Dev. 34(1); Muller et al., Handbook of Floating-Point Arithmetic, the
// theorem on Newton-Raphson based division).  tests/host/div_exact_check.cpp
// compares it with IEEE division on every fp32 significand of x for the
// divisors whose reciprocal rounds worst.
__host__ __device__ __forceinline__ float div_exact(float x, float s, float r) {
    const float q0 = x * r;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0);
    return __builtin_fmaf(__builtin_fmaf(-q1, s, x), r, q1);
}

// div_sqrt_dim of 8 values with one test per row: the three operations when
// every |y_i| lies in [2^-100, FLT_MAX], else IEEE division for all 8.
// Returns whether every |y_i| lies in [2^-55, 2^55], so that every quotient
// (d in [f32(sqrt 8), f32(sqrt 512)]) lies in div_exact's range [2^-60, 2^60].
//
// F16IN: the rows were fp16 before the transform, so no test is made.  Every
// fp16 value is an integer multiple of 2^-24 below 2^16 in magnitude; sums,
// differences and sign flips of such values keep every fp32 intermediate a
// multiple of 2^-24 (below 1 such a value is exactly representable, above 1
// the rounding grid is coarser than 2^-24), and 128 of them stay below 2^24.
// So y is 0 or |y| in [2^-24, 2^24]: the three operations are exact, the
// quotients lie in [2^-29, 2^23] inside div_exact's range, and only y = -0
// comes out +0 (IEEE gives -0).  The callers that take F16IN only square the
// quotient or quantize it (E8 rounds +-0 and +-0 + d alike), so the sign of a
// zero never reaches their outputs.
template <bool F16IN = false>
__host__ __device__ __forceinline__ bool div_sqrt_dim8(float y[8], float d, float r) {
    if constexpr (F16IN) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float q0 = y[i] * r;
            const float e = __builtin_fmaf(-q0, d, y[i]);
            y[i] = __builtin_fmaf(e, r, q0);
        }
        return true;
    }
    float lo = __builtin_fabsf(y[0]), hi = lo;
#pragma unroll
    for (int i = 1; i < 8; i++) {
        lo = __builtin_fminf(lo, __builtin_fabsf(y[i]));
        hi = __builtin_fmaxf(hi, __builtin_fabsf(y[i]));
    }
    if (lo >= 0x1p-100f && hi <= 0x1.fffffep127f) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float q0 = y[i] * r;
            const float e = __builtin_fmaf(-q0, d, y[i]);
            y[i] = __builtin_fmaf(e, r, q0);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) y[i] = y[i] / d;
    }
    return lo >= 0x1p-55f && hi <= 0x1p55f;
}

// rcp = RN(1 / div) (the caller's, computed once per launch).  Returns
// div_sqrt_dim8's range flag: forward (sign before the transform), every
// output lies in [2^-60, 2^60].  F16IN: as div_sqrt_dim8 (fp16 rows, the
// sign of a zero output unspecified).
template <bool F16IN = false>
__device__ __forceinline__ bool rht_lanes(float y[8], const float s[8], int part, int lpr, float div, float rcp,
                                          bool inverse) {
    if (!inverse) {
#pragma unroll
        for (int i = 0; i < 8; i++) y[i] = y[i] * s[i];
    }
    fwht_stages(y, part, lpr);
    const bool narrow = div_sqrt_dim8<F16IN>(y, div, rcp);
    if (inverse) {
#pragma unroll
        for (int i = 0; i < 8; i++) y[i] = y[i] * s[i];
    }
    return narrow;
}

__device__ __forceinline__ void load_signs8(const float* p, float s[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    s[0] = a.x; s[1] = a.y; s[2] = a.z; s[3] = a.w;
    s[4] = b.x; s[5] = b.y; s[6] = b.z; s[7] = b.w;
}

// -------------------------------------------------------------- dither ---
//
// Subtractive dither of the rotated path (build-defined: the reference has no
// E8 dither).  Vector v of a chunk with seed s gets d in [-1, 1)^8, uniform on
// a 2^-15 grid: a fundamental domain of 2Z^8, a sublattice of E8, so modulo E8
// the dither is uniform on the Voronoi cell and the error Q(t + d) - d - t is
// uniform on the cell (on the grid's resolution) and independent of t.
// Coordinates 4p .. 4p + 3 are the four 16-bit fields (least significant
// first) of h_p = mix64(mix64(s) + 2 v + p), p = 0, 1, with mix64 the
// SplitMix64 output function (Steele, Lea, Flood 2014).  The quantizer adds d
// to x / scale; the decoder subtracts it from the lattice point before scaling.
__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// key = mix64(seed); d = dither of vector v (exact in fp32)
__device__ __forceinline__ void dither8(uint64_t key, int64_t v, float d[8]) {
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const uint64_t h = mix64(key + (uint64_t)v * 2u + (uint64_t)p);
        const uint32_t lo = (uint32_t)h, hi = (uint32_t)(h >> 32);
        d[4 * p + 0] = (float)((int32_t)(lo & 0xFFFFu) - (1 << 15)) * 0x1p-15f;
        d[4 * p + 1] = (float)((int32_t)(lo >> 16) - (1 << 15)) * 0x1p-15f;
        d[4 * p + 2] = (float)((int32_t)(hi & 0xFFFFu) - (1 << 15)) * 0x1p-15f;
        d[4 * p + 3] = (float)((int32_t)(hi >> 16) - (1 << 15)) * 0x1p-15f;
    }
}

// ---------------------------------------------------------------- rANS ---

__host__ __device__ __forceinline__ uint32_t enc_pack(uint32_t f, uint32_t cum) {
    const uint32_t bl = f ? 32u - (uint32_t)__builtin_clz(f) : 0u;   // bit length of f
    uint32_t nb = 11u - bl;
    return f | (cum << 11) | (nb << 21);
}
__host__ __device__ __forceinline__ uint32_t enc_f(uint32_t e) { return e & 0x7ffu; }
__host__ __device__ __forceinline__ uint32_t enc_c(uint32_t e) { return (e >> 11) & 0x3ffu; }
__host__ __device__ __forceinline__ uint32_t enc_nb(uint32_t e) { return (e >> 21) & 0xfu; }

// Encoder table entry of the parallel chunk encoder, for the reference's
// step (core/gpu_ans.py:124-128: shift x right, emitting its low bits, while
// x >= 2 f, then x = L (x // f) + cum + x % f): F | base << 16, with
// nb = 11 - bitlen(f), thr = f << nb (the renormalisation threshold, in
// [L, 2L)),
// F = nb * 2^11 - thr (as int16) and base = L + cum - f (< 2^11).  A step on a
// state x in [L, 2L) is
//   k = nb - 1 + (x >= thr) = (x + F) >> 11;   x = (x >> k) + base
// (x - thr lies in (-2^11, 2^11), so the shift leaves nb - 1 or nb), and
// each half-word is read in place: two instructions for k instead of a
// field extract, a compare and an add with carry.  F is sign-extended, so a
// single-symbol table (f = L, nb = 0) steps too: k = 0, x unchanged.
__host__ __device__ __forceinline__ uint32_t encx_of(uint32_t e) {
    const uint32_t f = enc_f(e), c = enc_c(e), nb = enc_nb(e);
    const int32_t F = (int32_t)(nb << 11) - (int32_t)(f << nb);
    return ((uint32_t)F & 0xffffu) | (((uint32_t)kL + c - f) << 16);
}
__host__ __device__ __forceinline__ uint32_t encx_k(uint32_t x, uint32_t e) {
    return (uint32_t)((int32_t)x + (int32_t)(int16_t)(e & 0xffffu)) >> 11;
}
__host__ __device__ __forceinline__ uint32_t encx_step(uint32_t x, uint32_t e, uint32_t* k_out) {
    const uint32_t k = encx_k(x, e);
    *k_out = k;
    return (x >> k) + (e >> 16);
}

// Interval step: every state in [lo, hi] encodes the symbol; the image is
// exact when the interval lies on one side of the renormalisation threshold
// (both ends take the same k), otherwise the whole image range of the
// symbol: (x >> k) covers [f, 2f), with nb = k of the upper end and
// f = thr >> nb = ((nb << 11) - F) >> nb.
__host__ __device__ __forceinline__ void hull_step(uint32_t& lo, uint32_t& hi, uint32_t e) {
    const uint32_t klo = encx_k(lo, e), khi = encx_k(hi, e), base = e >> 16;
    if (klo == khi) {
        lo = (lo >> klo) + base;
        hi = (hi >> klo) + base;
    } else {
        const uint32_t thr = (uint32_t)((int32_t)(khi << 11) - (int32_t)(int16_t)(e & 0xffffu));
        const uint32_t f = thr >> khi;
        lo = f + base;
        hi = 2u * f - 1u + base;
    }
}

// One encoder step (core/gpu_ans.py:124-128): k renormalisation bits leave
// through *k / *bits (low k bits of x), then x = L + cum + (x >> k) - f.
__device__ __forceinline__ uint32_t enc_step(uint32_t x, uint32_t e, uint32_t* k_out) {
    uint32_t f = enc_f(e), nb = enc_nb(e);
    uint32_t thr = f << nb;
    uint32_t k = nb - 1u + (x >= thr ? 1u : 0u);
    *k_out = k;
    return (x >> k) + (uint32_t)kL + enc_c(e) - f;
}

// Bit-length helper for x in [1, 2^31).
__device__ __forceinline__ uint32_t bitlen(uint32_t x) { return 32u - (uint32_t)__clz((int)x); }

}  // namespace lq
