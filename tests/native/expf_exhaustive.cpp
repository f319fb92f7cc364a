// Exhaustive check of leafhip::libm_expf (leaf_amd/csrc/libm_expf.h) against
// this machine's libm expf: every one of the 2^32 float bit patterns.
// Prints "mismatches <n> first <bits or none>" and exits 0 when n == 0.
// Usage: expf_exhaustive [threads]
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "../../leaf_amd/csrc/libm_expf.h"

static uint32_t bits_of(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
static float float_of(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

int main(int argc, char** argv) {
    unsigned threads = argc > 1 ? unsigned(std::atoi(argv[1])) : std::thread::hardware_concurrency();
    if (threads == 0) threads = 1;
    std::vector<unsigned long long> bad(threads, 0);
    std::vector<long long> first(threads, -1);
    std::vector<std::thread> pool;
    for (unsigned w = 0; w < threads; ++w)
        pool.emplace_back([&, w] {
            const unsigned long long total = 1ull << 32;
            const unsigned long long begin = total * w / threads, end = total * (w + 1) / threads;
            for (unsigned long long i = begin; i < end; ++i) {
                const float x = float_of(uint32_t(i));
                const float want = expf(x), got = leafhip::libm_expf(x);
                const bool same = bits_of(want) == bits_of(got) || (std::isnan(want) && std::isnan(got));
                if (!same) {
                    if (first[w] < 0) first[w] = (long long)i;
                    ++bad[w];
                }
            }
        });
    for (auto& t : pool) t.join();
    unsigned long long n = 0;
    long long f = -1;
    for (unsigned w = 0; w < threads; ++w) {
        n += bad[w];
        if (f < 0 && first[w] >= 0) f = first[w];
    }
    if (f >= 0) {
        const float x = float_of(uint32_t(f));
        std::printf("mismatches %llu first 0x%08llx x=%a libm=%a here=%a\n", n, (unsigned long long)f, x, expf(x),
                    leafhip::libm_expf(x));
    } else {
        std::printf("mismatches 0 first none\n");
    }
    return n == 0 ? 0 : 1;
}
