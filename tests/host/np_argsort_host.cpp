// Host build of the device's numpy.argsort restatement (lq_argsort.h) with a
// one-lane group, for tests/test_np_argsort_host.py, which compares it with
// numpy.argsort on tie-heavy inputs.  np_std_sort_check also compares the
// header's restatement of libstdc++'s std::sort (the fallback the quicksort
// takes when its depth budget is spent) with std::sort itself, on inputs
// that include ones driving introsort into its heap-sort branch (McIlroy's
// adversary).
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

#include "lq_argsort.h"

namespace {
struct SerialGroup {
    static int tid() { return 0; }
    static int size() { return 1; }
    static void sync() {}
    static constexpr bool kWave = false;
};
}  // namespace

extern "C" int np_argsort_host(const int64_t* keys, int64_t* out, int n) {
    if (n < 0 || n > 1028) return -1;
    std::vector<int64_t> k(keys, keys + n);
    std::vector<int16_t> a(n > 0 ? n : 1);
    lq::NpScratch ns;
    lq::np_argsort<SerialGroup>(k.data(), a.data(), n, &ns);
    for (int i = 0; i < n; i++) out[i] = a[i];
    return 0;
}

// Compares lq::np_std_sort with std::sort on `cases` inputs from `seed`;
// returns the number of mismatching cases (heap-sort branch inputs included).
extern "C" long np_std_sort_check(uint64_t seed, long cases) {
    std::mt19937_64 rng(seed);
    long bad = 0;
    for (long c = 0; c < cases; c++) {
        const int n = 2 + (int)(rng() % 1027);
        std::vector<int64_t> key(n);
        const int kind = (int)(c % 5);
        for (int i = 0; i < n; i++) {
            if (kind == 0) key[i] = -(int64_t)(rng() % 4);
            else if (kind == 1) key[i] = -(int64_t)(rng() % 64);
            else if (kind == 2) key[i] = (int64_t)(rng() % 3) - 1000 * (int64_t)(rng() % 2);
            else if (kind == 3) key[i] = (int64_t)(rng() >> 1);
            else key[i] = 0;
        }
        if (kind == 4) {
            // McIlroy's adversary ("A killer adversary for quicksort", 1999):
            // run std::sort with a comparator that fixes values only when it
            // must, then use the values it fixed as keys.  Such keys drive
            // introsort into its depth limit, so the heap-sort branch runs.
            const int64_t gas = n;
            std::vector<int64_t> val(n, gas);
            std::vector<int> ptr(n);
            for (int i = 0; i < n; i++) ptr[i] = i;
            int64_t nsolid = 0;
            int candidate = -1;
            std::sort(ptr.begin(), ptr.end(), [&](int x, int y) {
                if (val[x] == gas && val[y] == gas) {
                    if (x == candidate) val[x] = nsolid++;
                    else val[y] = nsolid++;
                }
                if (val[x] == gas) candidate = x;
                else if (val[y] == gas) candidate = y;
                return val[x] < val[y];
            });
            key = val;
        }
        std::vector<int16_t> a(n), b(n);
        for (int i = 0; i < n; i++) a[i] = b[i] = (int16_t)i;
        if (c % 3 == 1) {   // start from a permutation, as the fallback does
            std::shuffle(a.begin(), a.end(), rng);
            b = a;
        }
        int32_t stk[3 * lq::kNpStack];
        lq::np_std_sort(key.data(), a.data(), 0, n, stk);
        const int64_t* kp = key.data();
        std::sort(b.begin(), b.end(), [kp](int16_t x, int16_t y) { return kp[x] < kp[y]; });
        if (a != b) bad++;
    }
    return bad;
}
