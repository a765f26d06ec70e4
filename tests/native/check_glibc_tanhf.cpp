// Host harness: compares the device header's glibc_expm1f / glibc_tanhf /
// gelu_tanh_ref_order (sapient_amd/csrc/glibc_tanhf.h, compiled here for the
// host) with the host libm over every f32 input. Prints one line per function
// with its mismatch count; exits non-zero on any mismatch.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#include "glibc_tanhf.h"

static inline uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline bool same(float a, float b) { return bits(a) == bits(b) || (isnan(a) && isnan(b)); }

// GELU in the reference's operation order with the host libm's tanhf
// (crates/sapient-backends/cpu/src/kernels/elementwise.rs:120-127).
static float gelu_libm(float v) {
    const float S = 0.79788456f, C = 0.044715f;
    const float inner = S * (v + C * v * v * v);
    return 0.5f * v * (1.0f + tanhf(inner));
}

int main(int argc, char** argv) {
    const int nthreads = argc > 1 ? atoi(argv[1]) : 8;
    std::atomic<uint64_t> bad_e{0}, bad_t{0}, bad_g{0};
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; ++t) {
        pool.emplace_back([&, t] {
            uint64_t be = 0, bt = 0, bg = 0;
            for (uint64_t u = t; u < (1ull << 32); u += nthreads) {
                float x;
                uint32_t w = (uint32_t)u;
                memcpy(&x, &w, 4);
                if (!same(sph::glibc_expm1f(x), expm1f(x))) ++be;
                if (!same(sph::glibc_tanhf(x), tanhf(x))) ++bt;
                if (!same(sph::gelu_tanh_ref_order(x), gelu_libm(x))) ++bg;
            }
            bad_e += be; bad_t += bt; bad_g += bg;
        });
    }
    for (auto& th : pool) th.join();
    printf("expm1f mismatches %llu\ntanhf mismatches %llu\ngelu mismatches %llu\n",
           (unsigned long long)bad_e.load(), (unsigned long long)bad_t.load(), (unsigned long long)bad_g.load());
    return (bad_e || bad_t || bad_g) ? 1 : 0;
}
