// Host build of lq_device.h's div_exact (x / s in five operations given
// r = RN(1 / s), two Markstein corrections) against IEEE fp32 division.
// Power-of-two scaling of x or s leaves the five operations exact while every
// intermediate stays normal, so x and s in [1, 2) stand for the whole range
// [2^-60, 2^60]; the check covers, for every fp32 significand of x:
//   - the 768 divisors whose reciprocal RN(1 / s) rounds worst (error closest
//     to half an ulp: the case the correction steps must absorb),
//   - 128 seeded random divisors and the significands 1, 1 + 2^-23, 2 - 2^-23,
//     sqrt(2) and 1.5;
// then x and s at every pair of binades 2^-60 .. 2^60 on a stride of
// significands, the range's end points included.  Built with
// -ffp-contract=off like the kernels; exit status 0 and "0 mismatches" when
// every quotient matches bit for bit.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <thread>
#include <vector>

#include "lq_device.h"

static uint32_t bits_of(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
static float float_of(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

int main() {
    // reciprocal rounding error of every divisor significand, in ulps of the result
    std::vector<std::pair<double, uint32_t>> err(1u << 23);
    for (uint32_t m = 0; m < (1u << 23); m++) {
        const float s = float_of((127u << 23) | m), r = 1.0f / s;
        int e;
        std::frexp((double)r, &e);
        err[m] = {std::fabs((double)r - 1.0 / (double)s) / std::ldexp(1.0, e - 24), m};
    }
    const int worst = 768;
    std::partial_sort(err.begin(), err.begin() + worst, err.end(),
                      [](const auto& a, const auto& b) { return a.first > b.first; });
    std::vector<uint32_t> divs;
    for (int k = 0; k < worst; k++) divs.push_back(err[k].second);
    std::mt19937 g(12345);
    for (int k = 0; k < 128; k++) divs.push_back(g() & 0x7fffffu);
    for (float f : {1.0f, 0x1.000002p0f, 0x1.fffffep0f, 0x1.6a09e6p0f, 1.5f}) divs.push_back(bits_of(f) & 0x7fffffu);
    std::printf("worst reciprocal error %.9f ulp\n", err[0].first);

    const unsigned nt = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
    std::vector<long> bad(nt, 0), total(nt, 0);
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; t++)
        th.emplace_back([&, t] {
            long b = 0, n = 0;   // thread-local counts: no shared cache line in the loop
            for (size_t k = t; k < divs.size(); k += nt) {
                const float s = float_of((127u << 23) | divs[k]), r = 1.0f / s;
                for (uint32_t m = 0; m < (1u << 23); m++) {
                    const float x = float_of((127u << 23) | m);
                    n += 2;
                    b += bits_of(lq::div_exact(x, s, r)) != bits_of(x / s);
                    b += bits_of(lq::div_exact(-x, s, r)) != bits_of(-x / s);
                }
            }
            bad[t] = b;
            total[t] = n;
        });
    for (auto& x : th) x.join();
    long nbad = 0, ntot = 0;
    for (unsigned t = 0; t < nt; t++) { nbad += bad[t]; ntot += total[t]; }
    // every pair of binades of x and s in [2^-60, 2^60], end points included
    for (int ex = -60; ex <= 59; ex++)
        for (int es = -60; es <= 59; es++) {
            for (uint32_t m = (uint32_t)(ex * 131 + es * 7 + 4096) % 7919; m < (1u << 23); m += 7919) {
                const float x = std::ldexp(float_of((127u << 23) | m), ex);
                const float s = std::ldexp(float_of((127u << 23) | ((m * 2654435761u) & 0x7fffffu)), es);
                const float r = 1.0f / s;
                ntot++;
                if (bits_of(lq::div_exact(x, s, r)) != bits_of(x / s)) {
                    if (nbad < 5) std::printf("mismatch x=%a s=%a\n", x, s);
                    nbad++;
                }
            }
        }
    for (float x : {0x1p-60f, 0x1.fffffep-61f * 2.0f, 0x1p60f, 0x1.fffffep59f})
        for (float s : {0x1p-60f, 0x1p60f, 0x1.fffffep59f, 0x1.000002p-60f}) {
            ntot++;
            nbad += bits_of(lq::div_exact(x, s, 1.0f / s)) != bits_of(x / s);
        }
    std::printf("%ld checks, %ld mismatches\n", ntot, nbad);
    return nbad != 0;
}
