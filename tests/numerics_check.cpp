// Host build of kernrt_amd/csrc/numerics.hpp checked against glibc and the
// oracle's conversions. Compiled by tests/test_numerics.py with
// g++ -O2 -ffp-contract=off. Usage: numerics_check <stride> <threads>
// prints "expf_mismatch <n>" and "f16_mismatch <n>".
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#include "../kernrt_amd/csrc/numerics.hpp"

int main(int argc, char** argv) {
    uint64_t stride = argc > 1 ? strtoull(argv[1], 0, 0) : 1;
    int threads = argc > 2 ? atoi(argv[2]) : 1;
    std::atomic<uint64_t> bad_exp{0}, bad_f16{0}, checked{0};
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; t++) {
        pool.emplace_back([&, t] {
            uint64_t be = 0, bf = 0, n = 0;
            for (uint64_t u = (uint64_t)t * stride; u < (1ull << 32); u += stride * (uint64_t)threads) {
                float x = kr::u2f((uint32_t)u);
                float g = expf(x), m = kr::glibc_expf(x);
                if (kr::f2u(g) != kr::f2u(m) && !(g != g && m != m)) {
                    if (be < 4) fprintf(stderr, "expf x=%a glibc=%a ours=%a\n", x, g, m);
                    be++;
                }
                // f16 widening is exact IEEE widening on normal codes; check the
                // narrowing round-trips those codes exactly.
                uint16_t h = kr::f32_to_f16_bits(x);
                uint32_t e = (h >> 10) & 0x1f;
                if (e >= 1 && e <= 30) {
                    float back = kr::f16w(h);
                    uint16_t again = kr::f32_to_f16_bits(back);
                    if (again != h) bf++;
                }
                n++;
            }
            bad_exp += be;
            bad_f16 += bf;
            checked += n;
        });
    }
    for (auto& th : pool) th.join();
    printf("checked %llu\nexpf_mismatch %llu\nf16_mismatch %llu\n", (unsigned long long)checked.load(),
           (unsigned long long)bad_exp.load(), (unsigned long long)bad_f16.load());
    return 0;
}
