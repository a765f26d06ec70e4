// Host harness: compares the device header's glibc_expf and the SiLU and
// erf-GELU expressions built on it (sapient_amd/csrc/glibc_expf.h, compiled
// here for the host) with the host libm over every f32 input. Prints one line
// per function with its mismatch count; exits non-zero on any mismatch.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#include "glibc_expf.h"

static inline uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline bool same(float a, float b) { return bits(a) == bits(b) || (isnan(a) && isnan(b)); }

// The reference's expressions with the host libm's expf
// (crates/sapient-backends/cpu/src/kernels/elementwise.rs:135-143, :163-174).
static float silu_libm(float v) { return v / (1.0f + expf(-v)); }
static float erf_libm(float x) {
    const float sign = isnan(x) ? x : copysignf(1.0f, x);
    x = fabsf(x);
    const float t = 1.0f / (1.0f + 0.3275911f * x);
    const float y = 1.0f - (0.25482959f + (-0.28449674f + (1.42141374f + (-1.45315203f + 1.06140543f * t) * t) * t) * t) *
                               t * expf(-x * x);
    return sign * y;
}
static float gelu_erf_libm(float v) { return 0.5f * v * (1.0f + erf_libm(v * 0.70710678118654752440f)); }

int main(int argc, char** argv) {
    const int nthreads = argc > 1 ? atoi(argv[1]) : 8;
    constexpr sph::Exp2fTable table = sph::exp2f_table();
    std::atomic<uint64_t> bad_e{0}, bad_n{0}, bad_s{0}, bad_g{0};
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; ++t) {
        pool.emplace_back([&, t] {
            uint64_t be = 0, bn = 0, bs = 0, bg = 0;
            for (uint64_t u = t; u < (1ull << 32); u += nthreads) {
                float x;
                uint32_t w = (uint32_t)u;
                memcpy(&x, &w, 4);
                if (!same(sph::glibc_expf_tab(x, table.tab), expf(x))) ++be;
                if ((w >> 31 || isnan(x)) && !same(sph::glibc_expf_nonpos_tab(x, table.tab), expf(x))) ++bn;
                if (!same(sph::silu_ref_order(x, table.tab), silu_libm(x))) ++bs;
                if (!same(sph::gelu_erf_ref_order(x, table.tab), gelu_erf_libm(x))) ++bg;
            }
            bad_e += be; bad_n += bn; bad_s += bs; bad_g += bg;
        });
    }
    for (auto& th : pool) th.join();
    printf("expf mismatches %llu\nexpf_nonpos mismatches %llu\nsilu mismatches %llu\ngelu_erf mismatches %llu\n",
           (unsigned long long)bad_e.load(), (unsigned long long)bad_n.load(), (unsigned long long)bad_s.load(),
           (unsigned long long)bad_g.load());
    return (bad_e || bad_n || bad_s || bad_g) ? 1 : 0;
}
