// CPU check of index-tts-25-metal_amd/csrc/glibc_math.h against the C library it restates:
// for fn in {expf, exp, logf}, counts the float inputs (bit patterns first + i * stride,
// i < count) whose result differs in any bit from glibc's expf(x), exp((double)x), logf(x).
// NaN inputs are skipped, and two NaN results agree whatever their bits (logf of a negative:
// the sampler only takes the log of a sum >= 1).
// Built by tests/test_libm_repro.py with g++ -O2 -ffp-contract=off -fopenmp.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "glibc_math.h"

int main(int argc, char** argv) {
    if (argc != 5) return 2;
    const int fn = std::atoi(argv[1]);
    const uint64_t first = std::strtoull(argv[2], nullptr, 0), stride = std::strtoull(argv[3], nullptr, 0),
                   count = std::strtoull(argv[4], nullptr, 0);
    uint64_t mismatches = 0, checked = 0;
#pragma omp parallel for reduction(+ : mismatches, checked) schedule(static)
    for (uint64_t i = 0; i < count; ++i) {
        const uint32_t b = static_cast<uint32_t>(first + i * stride);
        float x;
        std::memcpy(&x, &b, 4);
        if (std::isnan(x)) continue;
        ++checked;
        bool same;
        if (fn == 0) {
            const float a = itts::libm::expf_glibc(x), g = expf(x);
            same = std::memcmp(&a, &g, 4) == 0;
        } else if (fn == 1) {
            const double a = itts::libm::exp_glibc(static_cast<double>(x)), g = exp(static_cast<double>(x));
            same = std::memcmp(&a, &g, 8) == 0;
        } else {
            const float a = itts::libm::logf_glibc(x), g = logf(x);
            same = std::memcmp(&a, &g, 4) == 0 || (std::isnan(a) && std::isnan(g));
        }
        mismatches += same ? 0 : 1;
    }
    std::printf("%llu %llu\n", static_cast<unsigned long long>(checked), static_cast<unsigned long long>(mismatches));
    return 0;
}
