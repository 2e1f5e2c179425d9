// Compares expf_glibc (peregrine_amd/csrc/expf_glibc.h, the function the
// kernels call) with the host's libm expf over a range of f32 bit patterns.
// Usage: expf_sweep STEP THREADS -> prints "checked N mismatches M".
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>
#include <thread>
#include <vector>

#include "../../peregrine_amd/csrc/expf_glibc.h"

int main(int argc, char **argv) {
    const uint64_t step = argc > 1 ? strtoull(argv[1], nullptr, 0) : 1;
    const int nt = argc > 2 ? atoi(argv[2]) : 8;
    std::atomic<uint64_t> bad{0}, seen{0};
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++)
        th.emplace_back([&, t] {
            uint64_t b = 0, n = 0;
            for (uint64_t u = (uint64_t)t * step; u < (1ull << 32); u += step * (uint64_t)nt) {
                const uint32_t bits = (uint32_t)u;
                float x;
                memcpy(&x, &bits, 4);
                const float a = expf(x), m = expf_glibc(x);
                n++;
                if (phip_expf::f32_bits(a) != phip_expf::f32_bits(m) && !(isnan(a) && isnan(m))) {
                    if (b < 4) fprintf(stderr, "x=%a libm=%a expf_glibc=%a\n", x, a, m);
                    b++;
                }
            }
            bad += b;
            seen += n;
        });
    for (auto &t : th) t.join();
    printf("checked %llu mismatches %llu\n", (unsigned long long)seen.load(), (unsigned long long)bad.load());
    return 0;
}
