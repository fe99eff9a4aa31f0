// Host build of the parallel encoder's table entry and steps (lq_device.h:
// encx_of, encx_step, hull_step) against the reference's encoder step
// (core/gpu_ans.py:124-128): while x >= 2 f, emit the low bit of x and
// shift x right; then x = L (x // f) + cum + x % f.  Exhaustive over every
// frequency f in [1, L] and every state x in [L, 2L) for cum = 0 and
// cum = L - f (the base's extremes): the renormalisation bit count k (the
// emitted bits are the low k bits of x either way) and the next state.
// hull_step over [lo, hi] intervals (every pair for a stride of f, random
// pairs for the rest) against the reference step applied to every state of
// the interval: when all states take the same k, the image interval is
// exactly [min, max] of their images; otherwise it is the symbol's whole
// image range [L + cum, L + cum + f - 1], which holds every image.  Exit
// status 0 and "0 mismatches" when everything matches.
#include <cstdint>
#include <cstdio>
#include <random>

#include "lq_device.h"

namespace {
constexpr uint32_t L = LQ_L;

void ref_step(uint32_t x, uint32_t f, uint32_t cum, uint32_t* k, uint32_t* xn) {
    uint32_t n = 0;
    while (x >= 2 * f) {
        x >>= 1;
        n++;
    }
    *k = n;
    *xn = L * (x / f) + cum + x % f;
}
}  // namespace

int main() {
    long checks = 0, bad = 0;
    std::mt19937 g(7);
    for (uint32_t f = 1; f <= L; f++) {
        for (uint32_t cum : {0u, L - f}) {
            const uint32_t e = lq::encx_of(lq::enc_pack(f, cum));
            for (uint32_t x = L; x < 2 * L; x++) {
                uint32_t kr, xr, k;
                ref_step(x, f, cum, &kr, &xr);
                const uint32_t xn = lq::encx_step(x, e, &k);
                checks++;
                if (k != kr || xn != xr) {
                    if (bad < 5) std::printf("step f=%u cum=%u x=%u: k %u/%u x %u/%u\n", f, cum, x, k, kr, xn, xr);
                    bad++;
                }
            }
            // interval steps
            const int npairs = (f % 61 == 0) ? 0 : 64;
            auto check_interval = [&](uint32_t lo, uint32_t hi) {
                uint32_t k0, x0, kmin = 99, kmax = 0, imin = ~0u, imax = 0;
                for (uint32_t x = lo; x <= hi; x++) {
                    ref_step(x, f, cum, &k0, &x0);
                    kmin = k0 < kmin ? k0 : kmin;
                    kmax = k0 > kmax ? k0 : kmax;
                    imin = x0 < imin ? x0 : imin;
                    imax = x0 > imax ? x0 : imax;
                }
                uint32_t a = lo, b = hi;
                lq::hull_step(a, b, e);
                checks++;
                const bool ok = kmin == kmax ? (a == imin && b == imax)
                                             : (a == L + cum && b == L + cum + f - 1 && a <= imin && imax <= b);
                if (!ok) {
                    if (bad < 5) std::printf("hull f=%u cum=%u [%u,%u] -> [%u,%u], images [%u,%u]\n", f, cum, lo, hi, a, b,
                                             imin, imax);
                    bad++;
                }
            };
            if (npairs == 0) {   // every pair of one stride of states
                for (uint32_t lo = L; lo < 2 * L; lo += 37)
                    for (uint32_t hi = lo; hi < 2 * L; hi += 41) check_interval(lo, hi);
            } else {
                for (int p = 0; p < npairs; p++) {
                    uint32_t lo = L + g() % L, hi = L + g() % L;
                    if (lo > hi) { const uint32_t t = lo; lo = hi; hi = t; }
                    check_interval(lo, hi);
                }
            }
        }
    }
    std::printf("%ld checks, %ld mismatches\n", checks, bad);
    return bad != 0;
}
