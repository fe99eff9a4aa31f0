// Host build of lq_device.h's div_sqrt_dim (the rotation's division by
// f32(sqrt(D)) in three operations) against IEEE fp32 division: every fp32
// significand in [1, 4) for each divisor D = 8 .. 512, then zeros, subnormals,
// values around the 2^-100 threshold, values near the fp32 maximum, infinities
// and NaN.  Built with -ffp-contract=off like the kernels; exit status 0 and
// "0 mismatches" when every quotient matches bit for bit.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>

#include "lq_device.h"

static uint32_t bits_of(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
static float float_of(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

int main() {
    long bad = 0, total = 0;
    auto check = [&](float y, float d, float r) {
        const float want = y / d, got = lq::div_sqrt_dim(y, d, r);
        total++;
        if (bits_of(want) != bits_of(got) && !(std::isnan(want) && std::isnan(got))) {
            if (bad < 5) std::printf("mismatch y=%a d=%a: %a vs %a\n", y, d, got, want);
            bad++;
        }
    };
    for (int D = 8; D <= 512; D *= 2) {
        const float d = (float)std::sqrt((double)D), r = 1.0f / d;
        for (uint32_t m = 0; m < (1u << 23); m++)
            for (uint32_t e = 127; e <= 128; e++) {
                check(float_of((e << 23) | m), d, r);
                check(-float_of((e << 23) | m), d, r);
            }
        const float edge[] = {0.0f, -0.0f, 0x1p-149f, -0x1p-149f, 0x1p-126f, 0x1.fffffep-127f, 0x1p-100f,
                              0x1.fffffep-101f, 0x1.000002p-100f, 0x1p-90f, 3.0e38f, 0x1.fffffep127f,
                              -0x1.fffffep127f, std::numeric_limits<float>::infinity(),
                              -std::numeric_limits<float>::infinity(), std::numeric_limits<float>::quiet_NaN()};
        for (float y : edge) check(y, d, r);
        for (uint32_t m = 0; m < (1u << 23); m += 97) {   // subnormals and the smallest normals
            check(float_of(m), d, r);
            check(float_of((1u << 23) | m), d, r);
            check(float_of((27u << 23) | m), d, r);   // around 2^-100
            check(float_of((254u << 23) | m), d, r);  // the top binade
        }
    }
    // the 8-value form: rows mixing fast and fallback values take IEEE division for all
    {
        const float d = (float)std::sqrt(128.0), r = 1.0f / d;
        const float rows[4][8] = {{1.5f, -2.25f, 3.0f, 1e-3f, 7.0f, -0.5f, 100.0f, 2.0f},
                                  {1.5f, -0.0f, 3.0f, 1e-3f, 7.0f, -0.5f, 100.0f, 2.0f},
                                  {1.5f, 0x1p-120f, 3.0f, 1e-3f, 7.0f, -0.5f, 100.0f, 2.0f},
                                  {1.5f, 2.0f, std::numeric_limits<float>::infinity(), 1.0f, 7.0f, -0.5f, 1.0f, 2.0f}};
        for (const auto& row : rows) {
            float y[8];
            for (int i = 0; i < 8; i++) y[i] = row[i];
            lq::div_sqrt_dim8(y, d, r);
            for (int i = 0; i < 8; i++) {
                total++;
                if (bits_of(y[i]) != bits_of(row[i] / d)) bad++;
            }
        }
        for (uint32_t m = 0; m < (1u << 23); m += 8) {
            float y[8], x[8];
            for (int i = 0; i < 8; i++) x[i] = y[i] = float_of((127u << 23) | (m + i)) * ((i & 1) ? -1.0f : 1.0f);
            lq::div_sqrt_dim8(y, d, r);
            for (int i = 0; i < 8; i++) {
                total++;
                if (bits_of(y[i]) != bits_of(x[i] / d)) bad++;
            }
        }
    }
    std::printf("%ld checks, %ld mismatches\n", total, bad);
    return bad != 0;
}
