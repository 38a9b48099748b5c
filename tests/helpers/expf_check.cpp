// Host check of hy_expf (hymt2_amd/csrc/hy_expf.h) against the C library's expf over every
// float in [lo, hi] (both signs' bit patterns walked). Prints "mismatches=<n> total=<m>".
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "hy_expf.h"

int main(int argc, char** argv) {
    const float lo = argc > 1 ? strtof(argv[1], nullptr) : -105.f;
    const float hi = argc > 2 ? strtof(argv[2], nullptr) : 90.f;
    const int nth = argc > 3 ? atoi(argv[3]) : 8;
    std::vector<long> mism(nth, 0), total(nth, 0);
    std::vector<std::thread> th;
    for (int t = 0; t < nth; t++)
        th.emplace_back([&, t]() {
            for (uint64_t u = t; u < (1ull << 32); u += nth) {
                const uint32_t b = (uint32_t)u;
                float x;
                memcpy(&x, &b, 4);
                if (!(x >= lo && x <= hi)) continue;
                const float a = hy_expf(x), r = expf(x);
                uint32_t ba, br;
                memcpy(&ba, &a, 4);
                memcpy(&br, &r, 4);
                total[t]++;
                if (ba != br) mism[t]++;
            }
        });
    for (auto& x : th) x.join();
    long m = 0, n = 0;
    for (int t = 0; t < nth; t++) {
        m += mism[t];
        n += total[t];
    }
    printf("mismatches=%ld total=%ld\n", m, n);
    return m == 0 ? 0 : 1;
}
