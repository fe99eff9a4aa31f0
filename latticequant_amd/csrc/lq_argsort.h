// numpy.argsort order for int64 keys, restated for a cooperative group of
// lanes over LDS arrays (also built for the host, with one lane, by
// tests/host/np_argsort_host.cpp, which is checked against numpy.argsort).
//
// Why: build_rans_table ranks symbols by np.argsort(-counts) and
// np.argsort(-freqs) (reference core/gpu_ans.py:76,80).  numpy's default
// argsort is not stable, so which members of a tie group come first decides
// which frequencies the adjustment loop (core/gpu_ans.py:73-84) changes.
//
// numpy 2.x on an x86 host with AVX-512 sorts 64-bit integer keys with
// x86-simd-sort's argsort (a third-party library vendored by numpy; the
// algorithm below is restated from its published description and pinned by
// comparison with numpy.argsort itself):
//   argsort(key, n):  arg = 0 .. n-1;  if n > 1: qsort(0, n - 1, 2 * floor(log2 n))
//   qsort(l, r, it):
//     it <= 0            -> std::sort(arg[l .. r], key less), libstdc++ introsort
//     r + 1 - l <= 256   -> bitonic network over 8-lane registers (net_sort)
//     pivot = 5th smallest of key[arg[l + j * ((r - l) / 8)]], j = 1 .. 8
//     p = partition(l, r + 1, pivot): keys < pivot to the left, >= pivot to
//         the right, by 8-lane compress stores over blocks of 4 registers
//     qsort(l, p - 1, it - 1) unless pivot is the range minimum;
//     qsort(p, r, it - 1)     unless pivot is the range maximum.
// The two recursive calls touch disjoint ranges, so the order in which they
// run does not change the result; an explicit stack replaces the recursion.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lq {

// Network comparator: the larger key moves up; equal keys stay in place.
__host__ __device__ __forceinline__ void np_cmpx(int64_t* k, int16_t* a, int p, int q) {
    const int64_t kp = k[p], kq = k[q];
    if (kp > kq) {
        k[p] = kq; k[q] = kp;
        const int16_t t = a[p]; a[p] = a[q]; a[q] = t;
    }
}

// first lane of each of the 4 comparators of an in-register stage with partner i ^ m
__host__ __device__ __forceinline__ int np_pair_lane(int m, int p) {
    switch (m) {
        case 1: return 2 * p;                                 // 0 2 4 6
        case 2: case 3: return (p & 1) | ((p >> 1) << 2);     // 0 1 4 5
        default: return p;                                    // m = 4, 7: 0 1 2 3
    }
}

template <typename G>
__host__ __device__ void np_reg_stage(int64_t* k, int16_t* a, int nv, int m) {
    for (int t = G::tid(); t < nv * 4; t += G::size()) {
        const int reg = t >> 2, i = np_pair_lane(m, t & 3);
        np_cmpx(k, a, reg * 8 + i, reg * 8 + (i ^ m));
    }
    G::sync();
}

// The argsort network for n <= 256 (x86-simd-sort's argsort_n): the n
// (key, arg) pairs in k[0 .. n), a[0 .. n) are padded to nv registers of 8
// lanes (nv the least power of two with 8 nv >= n) with the type maximum,
// each register is sorted, then registers are merged by bitonic mirror and
// half-cleaner stages.  Results in k[0 .. n), a[0 .. n); k, a hold 8 nv entries.
template <typename G>
__host__ __device__ void np_net_sort(int64_t* k, int16_t* a, int n) {
    int nv = 1;
    while (nv * 8 < n) nv *= 2;
    for (int i = n + G::tid(); i < nv * 8; i += G::size()) { k[i] = INT64_MAX; a[i] = -1; }
    G::sync();
    np_reg_stage<G>(k, a, nv, 1);   // sort each register: partners i^1, i^3, i^1, i^7, i^2, i^1
    np_reg_stage<G>(k, a, nv, 3);
    np_reg_stage<G>(k, a, nv, 1);
    np_reg_stage<G>(k, a, nv, 7);
    np_reg_stage<G>(k, a, nv, 2);
    np_reg_stage<G>(k, a, nv, 1);
    for (int per = 2; per <= nv; per *= 2) {
        for (int t = G::tid(); t < nv * 4; t += G::size()) {   // mirror compare across registers
            const int grp = t / (per * 4), rem = t % (per * 4);
            const int i = rem / 8, l = rem % 8, off = grp * per;
            np_cmpx(k, a, 8 * (off + i) + l, 8 * (off + per - 1 - i) + 7 - l);
        }
        G::sync();
        for (int num = per / 2; num >= 2; num /= 2) {               // register half cleaners
            for (int t = G::tid(); t < nv * 4; t += G::size()) {
                const int grp = t / (per * 4), rem = t % (per * 4);
                const int l = rem % 8, q = rem / 8;
                const int jj = q / (num / 2), i = q % (num / 2);
                const int r1 = grp * per + jj * num + i;
                np_cmpx(k, a, 8 * r1 + l, 8 * (r1 + num / 2) + l);
            }
            G::sync();
        }
        np_reg_stage<G>(k, a, nv, 4);
        np_reg_stage<G>(k, a, nv, 2);
        np_reg_stage<G>(k, a, nv, 1);
    }
}

__host__ __device__ __forceinline__ int np_ilog2(int n) {   // floor(log2 n), n >= 1
    int l = 0;
    while ((n >> (l + 1)) != 0) l++;
    return l;
}
__host__ __device__ __forceinline__ int np_popc8(unsigned m) {
    m &= 0xffu;
    m = (m & 0x55u) + ((m >> 1) & 0x55u);
    m = (m & 0x33u) + ((m >> 2) & 0x33u);
    return (int)((m & 0x0fu) + (m >> 4));
}
__host__ __device__ __forceinline__ void np_swap(int16_t* a, int i, int j) {
    const int16_t t = a[i]; a[i] = a[j]; a[j] = t;
}

// ------------------------------------------------ libstdc++ std::sort --
// std::sort(first, last, key less) as libstdc++ implements it (introsort:
// median-of-three pivot moved to *first, unguarded Hoare partition, ranges
// of <= 16 left for one final insertion sort, heap sort once the depth limit
// 2 floor(log2 n) is spent).  Serial; stk holds 3 * 32 ints.

__host__ __device__ inline void np_adjust_heap(const int64_t* key, int16_t* a, int first, int hole, int len,
                                               int16_t value) {
    const int top = hole;
    int child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (key[a[first + child]] < key[a[first + child - 1]]) child--;
        a[first + hole] = a[first + child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        a[first + hole] = a[first + child - 1];
        hole = child - 1;
    }
    int parent = (hole - 1) / 2;   // push_heap
    while (hole > top && key[a[first + parent]] < key[value]) {
        a[first + hole] = a[first + parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    a[first + hole] = value;
}

__host__ __device__ inline void np_heap_sort(const int64_t* key, int16_t* a, int first, int last) {
    const int len = last - first;
    if (len >= 2) {   // make_heap
        for (int parent = (len - 2) / 2;; parent--) {
            np_adjust_heap(key, a, first, parent, len, a[first + parent]);
            if (parent == 0) break;
        }
    }
    while (last - first > 1) {   // sort_heap: pop_heap(first, last - 1, last - 1)
        --last;
        const int16_t value = a[last];
        a[last] = a[first];
        np_adjust_heap(key, a, first, 0, last - first, value);
    }
}

__host__ __device__ inline void np_std_sort(const int64_t* key, int16_t* a, int first, int last, int32_t* stk) {
    if (last - first < 2) return;
    int sp = 0;
    stk[0] = first; stk[1] = last; stk[2] = 2 * np_ilog2(last - first);
    sp = 1;
    while (sp > 0) {
        --sp;
        int f = stk[3 * sp], l = stk[3 * sp + 1], d = stk[3 * sp + 2];
        while (l - f > 16) {
            if (d == 0) {
                np_heap_sort(key, a, f, l);
                break;
            }
            --d;
            const int mid = f + (l - f) / 2, x = f + 1, z = l - 1;   // move_median_to_first(f, f+1, mid, l-1)
            const int64_t kx = key[a[x]], ky = key[a[mid]], kz = key[a[z]];
            int m;
            if (kx < ky) m = ky < kz ? mid : (kx < kz ? z : x);
            else m = kx < kz ? x : (ky < kz ? z : mid);
            np_swap(a, f, m);
            const int64_t kp = key[a[f]];   // unguarded_partition(f + 1, l, pivot = *f)
            int lo = f + 1, hi = l;
            while (true) {
                while (key[a[lo]] < kp) ++lo;
                --hi;
                while (kp < key[a[hi]]) --hi;
                if (!(lo < hi)) break;
                np_swap(a, lo, hi);
                ++lo;
            }
            if (sp < 32) {   // introsort_loop(cut, l, d); depth <= 2 log2(1028) + 1 frames
                stk[3 * sp] = lo; stk[3 * sp + 1] = l; stk[3 * sp + 2] = d;
                ++sp;
            }
            l = lo;
        }
    }
    // final insertion sort: guarded over the first 16, unguarded after
    // (the bound checks below never fire on a range introsort has prepared)
    const int g = last - first > 16 ? first + 16 : last;
    for (int i = first + 1; i < g; ++i) {
        const int16_t v = a[i];
        if (key[v] < key[a[first]]) {
            for (int j = i; j > first; --j) a[j] = a[j - 1];
            a[first] = v;
        } else {
            int j = i;
            while (j > first && key[v] < key[a[j - 1]]) { a[j] = a[j - 1]; --j; }
            a[j] = v;
        }
    }
    for (int i = g; i < last; ++i) {
        const int16_t v = a[i];
        int j = i;
        while (j > first && key[v] < key[a[j - 1]]) { a[j] = a[j - 1]; --j; }
        a[j] = v;
    }
}

// ------------------------------------------------------ quicksort part --

constexpr int kNpStack = 32;                       // qsort frames (depth <= 2 log2(1028) + 1)
constexpr int kNpScratchInts = 3 * kNpStack * 2 + 4;

// Per-group LDS scratch of np_argsort.
struct NpScratch {
    int64_t k[256];                 // network keys
    int16_t a[256];                 // network args; partition register blocks
    int32_t s[kNpScratchInts];      // qsort frames | introsort frames | scalars
};

// Compress stores of nvec 8-lane registers of args (regs[8 nvec]) around the
// pivot, in register order (x86-simd-sort's partition_vec per register):
// the keys < pivot of a register go to arg[l_store ...] in lane order, the
// keys >= pivot to the top of arg[.. r_store + 8) in lane order.  Every lane
// of the group evaluates all masks, so l_store / r_store stay uniform.
template <typename G>
__host__ __device__ __forceinline__ unsigned np_ge_mask(const int64_t* key, const int16_t* reg, int64_t pivot) {
    unsigned m = 0;
    for (int j = 0; j < 8; j++) m |= (key[reg[j]] >= pivot ? 1u : 0u) << j;
    return m;
}

template <typename G>
__host__ __device__ void np_store_regs(const int64_t* key, int16_t* arg, const int16_t* regs, int nvec,
                                       int64_t pivot, int& l_store, int& r_store, int32_t* flag_gt) {
    for (int t = G::tid(); t < 8 * nvec; t += G::size()) {
        const int v = t >> 3, j = t & 7;
        int ls = l_store, re = r_store + 8;
        for (int u = 0; u < v; u++) {
            const int gt = np_popc8(np_ge_mask<G>(key, regs + 8 * u, pivot));
            ls += 8 - gt;
            re -= gt;
        }
        const unsigned m = np_ge_mask<G>(key, regs + 8 * v, pivot);
        const unsigned below = (1u << j) - 1u;
        const int16_t x = regs[t];
        if ((m >> j) & 1u) {
            arg[re - np_popc8(m) + np_popc8(m & below)] = x;
            if (key[x] > pivot) *flag_gt = 1;
        } else {
            arg[ls + np_popc8(~m & below)] = x;
        }
    }
    for (int v = 0; v < nvec; v++) {
        const int gt = np_popc8(np_ge_mask<G>(key, regs + 8 * v, pivot));
        l_store += 8 - gt;
        r_store -= gt;
    }
    G::sync();
}

// x86-simd-sort's unrolled argsort partition (4 registers of 8 lanes per
// step) of arg[left .. right), right - left > 256.  Returns the first index
// of the >= pivot part; s[0] = 1 if some key in the range exceeds the pivot.
template <typename G>
__host__ __device__ int np_partition(const int64_t* key, int16_t* arg, int left, int right, int64_t pivot,
                                     int16_t* buf, int32_t* s) {
    constexpr int kB = 32;   // 4 registers x 8 lanes
    if (G::tid() == 0) {     // the range length is made a multiple of kB, serially
        int flag = 0;
        for (int i = (right - left) % kB; i > 0; --i) {
            const int64_t v = key[arg[left]];
            if (v > pivot) flag = 1;
            if (!(v < pivot)) np_swap(arg, left, --right);
            else ++left;
        }
        s[0] = flag; s[1] = left; s[2] = right;
    }
    G::sync();
    left = s[1];
    right = s[2];
    if (left == right) return left;
    // the first and last 4 registers are partitioned at the end (buf[0 .. 64))
    for (int t = G::tid(); t < 2 * kB; t += G::size()) buf[t] = t < kB ? arg[left + t] : arg[right - 2 * kB + t];
    G::sync();
    int r_store = right - 8, l_store = left;
    left += kB;
    right -= kB;
    while (right - left != 0) {
        int src;
        if ((r_store + 8) - right < left - l_store) {   // fewer stored on the right: load from the right
            right -= kB;
            src = right;
        } else {
            src = left;
            left += kB;
        }
        for (int t = G::tid(); t < kB; t += G::size()) buf[2 * kB + t] = arg[src + t];
        G::sync();
        np_store_regs<G>(key, arg, buf + 2 * kB, 4, pivot, l_store, r_store, &s[0]);
    }
    np_store_regs<G>(key, arg, buf, 8, pivot, l_store, r_store, &s[0]);   // left registers, then right
    return l_store;
}

// Sort arg[l .. l + len) (len <= 256) by key with the argsort network.
template <typename G>
__host__ __device__ void np_net_range(const int64_t* key, int16_t* arg, int len, NpScratch* ns) {
    if (len <= 1) return;
    for (int i = G::tid(); i < len; i += G::size()) {
        const int16_t x = arg[i];
        ns->a[i] = x;
        ns->k[i] = key[x];
    }
    G::sync();
    np_net_sort<G>(ns->k, ns->a, len);
    for (int i = G::tid(); i < len; i += G::size()) arg[i] = ns->a[i];
    G::sync();
}

// arg[0 .. n) = numpy.argsort(key[0 .. n)) for n <= 1028 (LDS arrays; every
// lane of the group calls it; uniform control flow).  Out of line: inlined
// into the table kernels its code costs them registers on every call path
// (the wave-per-stream table build measured 29 -> 53 us per C2 launch).
template <typename G>
__host__ __device__ __attribute__((noinline)) void np_argsort(const int64_t* key, int16_t* arg, int n, NpScratch* ns) {
    for (int i = G::tid(); i < n; i += G::size()) arg[i] = (int16_t)i;
    G::sync();
    if (n <= 1) return;
    int32_t* stk = ns->s;
    int32_t* istk = ns->s + 3 * kNpStack;
    int32_t* sc = ns->s + 6 * kNpStack;
    int sp = 1;   // uniform in every lane; frames live in LDS, written by lane 0
    if (G::tid() == 0) { stk[0] = 0; stk[1] = n - 1; stk[2] = 2 * np_ilog2(n); }
    G::sync();
    while (sp > 0) {
        --sp;
        const int l = stk[3 * sp], r = stk[3 * sp + 1], it = stk[3 * sp + 2];
        G::sync();   // every lane has read the frame before it is overwritten
        if (it <= 0) {
            if (G::tid() == 0) np_std_sort(key, arg, l, r + 1, istk);
            G::sync();
            continue;
        }
        if (r + 1 - l <= 256) {
            np_net_range<G>(key, arg + l, r + 1 - l, ns);
            continue;
        }
        int64_t smp[8];   // median of 8 samples: the 5th smallest (values only)
        const int step = (r - l) / 8;
#pragma unroll
        for (int j = 0; j < 8; j++) smp[j] = key[arg[l + (j + 1) * step]];
#pragma unroll
        for (int i = 0; i < 7; i++) {
#pragma unroll
            for (int j = 0; j < 7 - i; j++) {
                const int64_t x = smp[j], y = smp[j + 1];
                smp[j] = x < y ? x : y;
                smp[j + 1] = x < y ? y : x;
            }
        }
        const int64_t pivot = smp[4];
        const int p = np_partition<G>(key, arg, l, r + 1, pivot, ns->a, sc);
        const int any_gt = sc[0];
        G::sync();
        const bool go_left = p > l;   // pivot above the range minimum
        const bool go_right = any_gt != 0;   // pivot below the range maximum
        if (go_right && sp < kNpStack) {
            if (G::tid() == 0) { stk[3 * sp] = p; stk[3 * sp + 1] = r; stk[3 * sp + 2] = it - 1; }
            sp++;
        }
        if (go_left && sp < kNpStack) {
            if (G::tid() == 0) { stk[3 * sp] = l; stk[3 * sp + 1] = p - 1; stk[3 * sp + 2] = it - 1; }
            sp++;
        }
        G::sync();
    }
}

}  // namespace lq
