// Host-side check of the quantizer's nearest-point search (lq_device.h,
// e8_nearest_fast: estimate of d1 - d2 with an error margin, exact
// reference-order fallback) against the CPU oracle's encode_e8
// (oracle/lq_oracle.c, a restatement of core/e8_quantizer.py:20-83).
// The device functions are __host__ __device__; this file is built for the
// host only, with -ffp-contract=off like the kernels.
//
// Usage: e8_fast_check N   (N vectors per thread, 8 threads); exit status 0
// when every vector matches.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <thread>
#include <vector>
#include <atomic>

#include "lq_device.h"

extern "C" void lqo_encode_e8(const float* x, float* out, int64_t n);

namespace {
std::atomic<long> g_fail{0}, g_total{0};

bool same(const float x[8]) {
    float ic[8], ref[8];
    const int c = lq::e8_nearest_fast(x, ic);
    lqo_encode_e8(x, ref, 1);
    for (int i = 0; i < 8; i++) {
        const float v = ic[i] + (c ? 0.5f : 0.f);
        if (!(v == ref[i])) return false;
    }
    return true;
}

// Inputs: Gaussian at scales 2^-4 .. 2^19; points near the boundary between
// the D8 and D8 + 1/2 candidates (their midpoint, perturbed by 2^-k); dyadic
// grid points (exact ties); one large coordinate among small ones;
// half-integers perturbed by 2^-k.
void worker(uint64_t seed, long n) {
    std::mt19937_64 g(seed);
    std::normal_distribution<float> N(0.f, 1.f);
    std::uniform_real_distribution<float> U(-1.f, 1.f);
    float x[8];
    long fails = 0;
    for (long it = 0; it < n; it++) {
        const int kind = (int)(g() % 16);
        const float sc = std::ldexp(1.0f, (int)(g() % 24) - 4);
        if (kind < 6) {
            for (int i = 0; i < 8; i++) x[i] = N(g) * sc;
        } else if (kind < 11) {
            for (int i = 0; i < 8; i++) x[i] = N(g) * sc;
            float c1[8], c2[8], y[8];
            lq::d8_round(x, c1);
            for (int i = 0; i < 8; i++) y[i] = x[i] - 0.5f;
            lq::d8_round(y, c2);
            const float eps = std::ldexp(1.0f, -(int)(g() % 30));
            for (int i = 0; i < 8; i++) x[i] = 0.5f * (c1[i] + c2[i] + 0.5f) + (kind == 6 ? 0.f : U(g) * eps);
        } else if (kind < 13) {
            for (int i = 0; i < 8; i++) x[i] = (float)((int)(g() % 64) - 32) * 0.25f;
        } else if (kind < 14) {
            for (int i = 0; i < 8; i++) x[i] = N(g) * 1e-3f;
            x[g() % 8] = N(g) * sc * 100.f;
        } else {
            for (int i = 0; i < 8; i++)
                x[i] = (float)((int)(g() % 16) - 8) + 0.5f + U(g) * std::ldexp(1.0f, -(int)(g() % 26));
        }
        if (!same(x)) {
            if (fails < 5) {
                std::printf("mismatch (kind %d):", kind);
                for (int i = 0; i < 8; i++) std::printf(" %.9g", x[i]);
                std::printf("\n");
            }
            fails++;
        }
    }
    g_fail += fails;
    g_total += n;
}
}  // namespace

int main(int argc, char** argv) {
    const long n = argc > 1 ? std::atol(argv[1]) : 1000000;
    std::vector<std::thread> th;
    for (int t = 0; t < 8; t++) th.emplace_back(worker, 0x5eed0000u + t, n);
    for (auto& t : th) t.join();
    std::printf("checked %ld vectors, %ld mismatches\n", (long)g_total, (long)g_fail);
    return g_fail != 0;
}
