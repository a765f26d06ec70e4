// glibc_sincosf.h — f32 sin and cos evaluated exactly as glibc (2.28 and
// later) does on x86_64 CPUs with FMA.
//
// The reference's RoPE calls Rust's f32::sin and f32::cos
// (crates/sapient-backends/cpu/src/kernels/rope.rs:52-53, :125-126), which on
// x86_64-linux-gnu are glibc's sinf and cosf. glibc implements them with the
// algorithm of Szabolcs Nagy published in ARM's optimized-routines (glibc
// sysdeps/ieee754/flt-32/s_sinf.c, s_cosf.c, sincosf.h), all in double
// precision with one final rounding to f32:
//   |x| < 0.75 (top-12-bit compare against pi/4): the polynomial directly;
//   |x| < 120: x = n·pi/2 + r with n from x·(2/pi) (2^24-scaled, truncated,
//     rounded by adding 2^23 and shifting), r = x − n·pi/2;
//   larger: an integer multiply of the mantissa by 4/pi (192 bits, a table
//     sliding 8 bits per entry) gives n and r as a 2.62 fixed-point fraction.
// sin(r) ≈ r + r³·s1 + r⁷·(s2 + r²·s3) and cos(r) ≈ c0 + r²·c1 + r⁴·c2 +
// r⁶·(c3 + r²·c4); the quadrant picks sin or cos and the sign, the second
// coefficient set being the negated cosine. On a CPU with FMA the x86_64
// build selects the variant compiled with contraction (s_sinf-fma.c,
// s_cosf-fma.c): every a + b·c of the polynomial and the reduction
// x − n·pi/2 is one fused multiply-add. That is what runs on current x86_64
// servers, so it is what is restated here.
//
// Declared __host__ __device__ so the test suite can compare this very code
// with the host libm over all 2^32 inputs.
//
// Provenance and licence: the algorithm and its constants (the polynomial
// coefficients, the 4/pi bit table) are those of ARM's optimized-routines
// (Copyright (c) 2018 Arm Limited; MIT OR Apache-2.0 WITH LLVM-exception), as
// carried by glibc (LGPL-2.1-or-later); they are restated here from the
// published algorithm, not copied from either source tree.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sph {

// 2/pi in hexadecimal, 0.A2F9836E 4E441529 FC2757D1 F534DDC0 DB629599 3C439041:
// entry i holds the 32-bit window of fraction bytes i-3 .. i, so a window
// starting at any byte is one aligned load.
struct InvPio4Table {
    uint32_t w[24];
};

__host__ __device__ constexpr InvPio4Table inv_pio4_table() {
    return {{0xa2u,       0xa2f9u,     0xa2f983u,   0xa2f9836eu, 0xf9836e4eu, 0x836e4e44u,
             0x6e4e4415u, 0x4e441529u, 0x441529fcu, 0x1529fc27u, 0x29fc2757u, 0xfc2757d1u,
             0x2757d1f5u, 0x57d1f534u, 0xd1f534ddu, 0xf534ddc0u, 0x34ddc0dbu, 0xddc0db62u,
             0xc0db6295u, 0xdb629599u, 0x6295993cu, 0x95993c43u, 0x993c4390u, 0x3c439041u}};
}

namespace sincosf_detail {

constexpr double kHpiInv = 0x1.45F306DC9C883p+23;  // 2/pi · 2^24
constexpr double kHpi = 0x1.921FB54442D18p0;       // pi/2
constexpr double kPi63 = 0x1.921FB54442D18p-62;    // pi/2 · 2^-62
constexpr double kC0 = 0x1p0, kC1 = -0x1.ffffffd0c621cp-2, kC2 = 0x1.55553e1068f19p-5,
                 kC3 = -0x1.6c087e89a359dp-10, kC4 = 0x1.99343027bf8c3p-16;
constexpr double kS1 = -0x1.555545995a603p-3, kS2 = 0x1.1107605230bc4p-7, kS3 = -0x1.994eb3774cf24p-13;

__host__ __device__ inline uint32_t abstop12(float x) { return (__builtin_bit_cast(uint32_t, x) >> 20) & 0x7ffu; }

// sin(x) for even n, ±cos(x) for odd n (neg_cos: the negated cosine set).
__host__ __device__ inline float poly(double x, double x2, bool neg_cos, int n) {
    if ((n & 1) == 0) {
        const double x3 = x * x2;
        const double s1 = __builtin_fma(x2, kS3, kS2);
        const double x7 = x3 * x2;
        const double s = __builtin_fma(x3, kS1, x);
        return (float)__builtin_fma(x7, s1, s);
    }
    const double g = neg_cos ? -1.0 : 1.0;
    const double x4 = x2 * x2;
    const double c2 = __builtin_fma(x2, g * kC4, g * kC3);
    const double c1 = __builtin_fma(x2, g * kC1, g * kC0);
    const double x6 = x4 * x2;
    const double c = __builtin_fma(x4, g * kC2, c1);
    return (float)__builtin_fma(x6, c2, c);
}

// |x| < 120: r = x − n·pi/2 with n = round(x·2/pi) formed as glibc's
// non-intrinsic build does it (truncate the 2^24-scaled product, add 2^23,
// arithmetic shift by 24).
__host__ __device__ inline double reduce_fast(double x, int* np) {
    const double r = x * kHpiInv;
    const int n = ((int32_t)r + 0x800000) >> 24;
    *np = n;
    return __builtin_fma(-(double)n, kHpi, x);
}

// |x| >= 120: the mantissa times the 96 bits of 4/pi that matter at this
// exponent gives the 2.62 fixed-point fraction of x / (pi/2); n is its
// rounded integer part, the rest is converted to double and scaled by pi/2.
__host__ __device__ inline double reduce_large(uint32_t xi, int* np, const uint32_t* inv_pio4) {
    const uint32_t* arr = inv_pio4 + ((xi >> 26) & 15u);
    const int shift = (int)((xi >> 23) & 7u);
    uint32_t m = (xi & 0xffffffu) | 0x800000u;
    m <<= shift;
    uint64_t res0 = (uint64_t)(uint32_t)(m * arr[0]);
    const uint64_t res1 = (uint64_t)m * arr[4];
    const uint64_t res2 = (uint64_t)m * arr[8];
    res0 = (res2 >> 32) | (res0 << 32);
    res0 += res1;
    const uint64_t n = (res0 + (1ull << 61)) >> 62;
    res0 -= n << 62;
    const double x = (double)(int64_t)res0;
    *np = (int)n;
    return x * kPi63;
}

}  // namespace sincosf_detail

// sinf(y) and cosf(y) at once, each bit-identical to glibc's. glibc branches
// three ways on |y|; here:
//  - below 0.75 glibc evaluates the polynomials on y itself; the fast
//    reduction gives n = 0 and r = fma(-0, pi/2, y) = y exactly there, with
//    the quadrant signs and coefficient set of n = 0 — the same evaluation,
//    so the two lower branches collapse into one;
//  - below 2^-12 glibc returns y and 1.0f (kept as a select: the
//    polynomials round to the same values except sin(-0), which they make +0);
//  - for |y| >= 120 the large reduction replaces the fast one (its quadrant
//    also absorbs the sign). On the GPU this is a branch a wave skips when
//    none of its lanes holds such an argument, so callers that give a wave
//    angles of similar size pay for the large reduction only where it is used.
// sincosf_poly and sinf_poly/cosf_poly evaluate identical expressions, so
// one pair of polynomials serves both results.
__host__ __device__ inline void glibc_sincosf_tab(float y, const uint32_t* inv_pio4, float* sin_out, float* cos_out) {
    using namespace sincosf_detail;
    const uint32_t top = abstop12(y);
    if (top >= abstop12(__builtin_inff())) {  // inf, NaN: NaN
        *sin_out = *cos_out = (y - y) / (y - y);
        return;
    }
    const uint32_t xi = __builtin_bit_cast(uint32_t, y);
    int n;
    double x;
    int q;  // quadrant of the signs and coefficient set
    if (top >= abstop12(120.0f)) {
        x = reduce_large(xi, &n, inv_pio4);
        q = n + (int)(xi >> 31);
    } else {
        x = reduce_fast((double)y, &n);
        q = n;
    }
    const double sgn = ((q + 1) & 2) ? -1.0 : 1.0;  // signs {1, -1, -1, 1} by q mod 4
    const double x2 = x * x;
    const float sp = poly(x * sgn, x2, false, 0);
    const float cp = poly(x * sgn, x2, (q & 2) != 0, 1);
    const bool tiny = top < abstop12(0x1p-12f);
    *sin_out = tiny ? y : ((n & 1) ? cp : sp);
    *cos_out = tiny ? 1.0f : ((n & 1) ? sp : cp);
}

}  // namespace sph
