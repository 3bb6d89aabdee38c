// Exhaustive check of wick::exp_f32 (wick_amd/csrc/exp_f32.h) against the C
// library's expf on this host: every one of the 2^32 f32 bit patterns, split
// over the threads given on the command line.  Prints the mismatch count and
// the first mismatching inputs; exit status 0 only when there are none.
#include "exp_f32.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

int main(int argc, char **argv) {
    const int nt = argc > 1 ? atoi(argv[1]) : 8;
    std::vector<unsigned long long> bad(nt, 0);
    std::vector<unsigned> first(nt, 0);
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++)
        th.emplace_back([&, t] {
            const unsigned long long lo = (1ULL << 32) * t / nt, hi = (1ULL << 32) * (t + 1) / nt;
            for (unsigned long long u = lo; u < hi; u++) {
                const unsigned v = (unsigned)u;
                float x;
                memcpy(&x, &v, 4);
                const float a = expf(x), b = wick::exp_f32(x);
                unsigned ua, ub;
                memcpy(&ua, &a, 4);
                memcpy(&ub, &b, 4);
                if (ua != ub && !(std::isnan(a) && std::isnan(b))) {
                    if (!bad[t]) first[t] = v;
                    bad[t]++;
                }
            }
        });
    unsigned long long total = 0;
    for (int t = 0; t < nt; t++) {
        th[t].join();
        total += bad[t];
        if (bad[t]) printf("first mismatch in slice %d: input bits 0x%08x\n", t, first[t]);
    }
    printf("mismatches over all 2^32 inputs: %llu\n", total);
    return total != 0;
}
