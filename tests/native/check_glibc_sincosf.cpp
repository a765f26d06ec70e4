// Host harness: compares the device header's glibc_sincosf_tab
// (sapient_amd/csrc/glibc_sincosf.h, compiled here for the host) with the host
// libm over every f32 input — with sinf and cosf called separately (through
// function pointers, so the compiler cannot merge them) and with sincosf,
// which is what a compiler may turn the reference's f32::sin_cos (rope.rs:52)
// into. Prints one line per function with its mismatch count and the first
// few mismatching inputs; exits non-zero on any mismatch.
#ifndef _GNU_SOURCE
#define _GNU_SOURCE  // sincosf
#endif
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <thread>
#include <vector>

#include "glibc_sincosf.h"

static inline uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline bool same(float a, float b) { return bits(a) == bits(b) || (isnan(a) && isnan(b)); }

static float (*volatile sin_fn)(float) = sinf;
static float (*volatile cos_fn)(float) = cosf;

int main(int argc, char** argv) {
    const int nthreads = argc > 1 ? atoi(argv[1]) : 8;
    constexpr sph::InvPio4Table table = sph::inv_pio4_table();
    std::atomic<uint64_t> bad_s{0}, bad_c{0};
    std::mutex mu;
    int shown = 0;
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; ++t) {
        pool.emplace_back([&, t] {
            uint64_t bs = 0, bc = 0;
            for (uint64_t u = t; u < (1ull << 32); u += nthreads) {
                float x;
                const uint32_t w = (uint32_t)u;
                memcpy(&x, &w, 4);
                float s, c;
                sph::glibc_sincosf_tab(x, table.w, &s, &c);
                const float rs = sin_fn(x), rc = cos_fn(x);
                float ps, pc;
                sincosf(x, &ps, &pc);
                const bool ok_s = same(s, rs) && same(s, ps), ok_c = same(c, rc) && same(c, pc);
                bs += !ok_s;
                bc += !ok_c;
                if (!(ok_s && ok_c)) {
                    std::lock_guard<std::mutex> lock(mu);
                    if (shown < 8) {
                        ++shown;
                        printf("x=%a (0x%08x): sin %a vs %a, cos %a vs %a\n", x, w, s, rs, c, rc);
                    }
                }
            }
            bad_s += bs;
            bad_c += bc;
        });
    }
    for (auto& th : pool) th.join();
    printf("sinf mismatches %llu\ncosf mismatches %llu\n", (unsigned long long)bad_s.load(),
           (unsigned long long)bad_c.load());
    return (bad_s || bad_c) ? 1 : 0;
}
