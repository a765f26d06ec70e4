// glibc_expf.h — f32 exp evaluated exactly as glibc (2.27 and later) does on
// x86_64 CPUs with FMA.
//
// The reference's SiLU and erf-GELU call Rust's f32::exp (elementwise.rs:137,
// :142, :172 in crates/sapient-backends/cpu/src/kernels/), which on
// x86_64-linux-gnu is glibc's expf. glibc implements it with the algorithm of
// Szabolcs Nagy published in ARM's optimized-routines (glibc
// sysdeps/ieee754/flt-32/e_expf.c): with N = 32,
//   x·N/ln2 = k + r, r ∈ [-1/2, 1/2], k an integer (round to nearest even),
//   exp(x) = 2^(k/N) · 2^(r/N) ≈ s · (C0 r³ + C1 r² + C2 r + 1),
// all in double precision, s = 2^((k mod N)/N) from a 32-entry table with the
// exponent bits of k/N added, then one rounding to f32. On a CPU with FMA the
// x86_64 build selects the variant compiled with contraction (e_expf-fma.c):
// the product x·N/ln2 is fused into both range-reduction steps and the three
// polynomial steps are fused multiply-adds. That is what runs on current
// x86_64 servers, so it is what is restated here; the non-FMA build differs
// from it on a handful of f32 inputs.
//
// Declared __host__ __device__ so the test suite can compare this very code
// with the host libm over all 2^32 inputs.
//
// Provenance and licence: the algorithm and its constants (the polynomial
// coefficients, the 2^(i/32) table) are those of ARM's optimized-routines
// (Copyright (c) 2017-2018 Arm Limited; MIT OR Apache-2.0 WITH LLVM-exception),
// as carried by glibc (LGPL-2.1-or-later); they are restated here from the
// published algorithm, not copied from either source tree.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sph {

// tab[i] = bits(RN(2^(i/32))) − (i << 47): adding k << 47 for k ≡ i (mod 32)
// yields the double 2^(k/32) exactly.
struct Exp2fTable {
    uint64_t tab[32];
};

__host__ __device__ constexpr Exp2fTable exp2f_table() {
    return {{
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
    }};
}

// expf with the 2^(i/32) table passed in: device code keeps it in LDS or
// registers, host code uses exp2f_table().
__host__ __device__ inline float glibc_expf_tab(float x, const uint64_t* tab) {
    // glibc branches to its special cases for |x| >= 88 or NaN: overflow above
    // 0x1.62e42ep6 and +inf give +inf, underflow below -0x1.9fe368p6 and -inf
    // give 0, NaN gives NaN, and the rest of that range falls through to the
    // main path. Here those are selects after the main path has run on x
    // clamped into [underflow bound, overflow bound] (a NaN passes through it
    // to a NaN; the table index is taken mod 32), so lanes never diverge.
    constexpr float kUnder = -0x1.9fe368p6f, kOver = 0x1.62e42ep6f;
    const bool under = x < kUnder, over = x > kOver;
    const float xc = under ? kUnder : (over ? kOver : x);
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;

    const double xd = (double)xc;
    // z = x·N/ln2 feeds two additions, and the contracting build fuses the
    // product into both: kd = RN(z + shift) rounds z to an integer (ties to
    // even) and r = z − k is formed from the exact product.
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    const double s = __builtin_bit_cast(double, t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return over ? __builtin_bit_cast(float, 0x7f800000u) : (under ? 0.0f : (float)y);
}

// glibc_expf_tab for a <= 0 or NaN (erf's exp(−x²)), written without
// branches: the special cases such arguments reach are −inf and underflow
// below −0x1.9fe368p6, both 0, and NaN; every other argument, −103.97 ≤ a < −88
// included, takes glibc's main path. The main path runs on the argument clamped
// at the underflow bound (its value is then discarded for 0) and carries a NaN
// through to a NaN (the table index stays in range: it is taken mod 32).
__host__ __device__ inline float glibc_expf_nonpos_tab(float a, const uint64_t* tab) {
    constexpr float kUnder = -0x1.9fe368p6f;
    const bool under = a < kUnder;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)(under ? kUnder : a);
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    const double s = __builtin_bit_cast(double, t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return under ? 0.0f : (float)y;
}

__host__ inline float glibc_expf(float x) {
    constexpr Exp2fTable t = exp2f_table();
    return glibc_expf_tab(x, t.tab);
}

// Reference operation orders, f32 with every step rounded on its own.

// SiLU (elementwise.rs:141-143): v / (1 + exp(-v)).
__host__ __device__ inline float silu_ref_order(float v, const uint64_t* tab) {
    return v / (1.0f + glibc_expf_tab(-v, tab));
}

// 1 / d for erf_ref_order's d = 1 + p·|x| (d >= 1, or +inf, or NaN). The
// device forms it from the hardware reciprocal and one FMA correction (4
// instructions against ~10 for the IEEE sequence); every f32 input of the
// erf-GELU kernel gives the IEEE result (tested on the GPU over all 2^32
// inputs). Past 2^64, where erf's exp(−x²) factor is exactly 0 and t only has
// to be finite, d is clamped so the correction never meets an infinity. The
// host build divides.
__host__ __device__ inline float recip_erf(float d) {
#if defined(__HIP_DEVICE_COMPILE__)
    d = d < 0x1p64f ? d : (d != d ? d : 0x1p64f);
    const float r = __builtin_amdgcn_rcpf(d);
    return __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
#else
    return 1.0f / d;
#endif
}

// Abramowitz-Stegun erf (elementwise.rs:163-174); signum(NaN) is NaN and
// signum(±0) is ±1, as Rust's f32::signum.
__host__ __device__ inline float erf_ref_order(float x, const uint64_t* tab) {
    const float sign = x != x ? x : __builtin_copysignf(1.0f, x);
    x = __builtin_fabsf(x);
    const float t = recip_erf(1.0f + 0.3275911f * x);
    const float poly =
        0.25482959f + (-0.28449674f + (1.42141374f + (-1.45315203f + 1.06140543f * t) * t) * t) * t;
    const float y = 1.0f - poly * t * glibc_expf_nonpos_tab(-x * x, tab);
    return sign * y;
}

// erf-GELU (elementwise.rs:135-138): 0.5 v (1 + erf(v / √2)).
__host__ __device__ inline float gelu_erf_ref_order(float v, const uint64_t* tab) {
    const float inv_sqrt2 = 0.70710678118654752440f;
    return 0.5f * v * (1.0f + erf_ref_order(v * inv_sqrt2, tab));
}

}  // namespace sph
