// glibc_tanhf.h — f32 tanh evaluated exactly as glibc 2.35 does.
//
// The reference's GELU calls Rust's f32::tanh (elementwise.rs:125 in
// crates/sapient-backends/cpu/src/kernels/), which on x86_64-linux-gnu is
// glibc's tanhf. glibc 2.35 implements tanhf and its helper expm1f with the
// fdlibm algorithms (sysdeps/ieee754/flt-32/s_tanhf.c, s_expm1f.c: Sun
// Microsystems fdlibm, float conversion by Cygnus Support). The functions
// below follow those published algorithms step for step in IEEE f32 — the
// same constants, the same operation order, every product and sum rounded on
// its own — so they return glibc's bits for every f32 input. That matters
// because GELU forms 1 + tanh(z), which cancels for z < -3: the reference's
// result there is glibc's rounding of tanh, and only the same bits reproduce
// it. The translation unit must be compiled with -ffp-contract=off.
//
// Declared __host__ __device__ so the test suite can compare the very same
// code against the host libm over all 2^32 inputs.
//
// Provenance and licence: the algorithms and constants are fdlibm's (Copyright
// (C) 1993 by Sun Microsystems, Inc.: "Permission to use, copy, modify, and
// distribute this software is freely granted, provided that this notice is
// preserved."; float conversion by Cygnus Support), as carried by glibc.
// They are restated here step for step from the published algorithm.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sph {

__host__ __device__ inline uint32_t fbits(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float bitsf(uint32_t u) { return __builtin_bit_cast(float, u); }

// fdlibm expm1f: exp(x) - 1.
__host__ __device__ inline float glibc_expm1f(float x) {
    const float o_threshold = 8.8721679688e+01f;  // 0x42b17180
    const float ln2_hi = 6.9313812256e-01f;       // 0x3f317180
    const float ln2_lo = 9.0580006145e-06f;       // 0x3717f7d1
    const float invln2 = 1.4426950216e+00f;       // 0x3fb8aa3b
    // rational-approximation coefficients of the primary range
    const float Q1 = -3.3333335072e-02f;  // 0xbd088889
    const float Q2 = 1.5873016091e-03f;   // 0x3ad00d01
    const float Q3 = -7.9365076090e-05f;  // 0xb8a670cd
    const float Q4 = 4.0082177293e-06f;   // 0x36867e54
    const float Q5 = -2.0109921195e-07f;  // 0xb457edbb

    uint32_t hx = fbits(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    float hi, lo, c = 0.0f, t;
    int32_t k;

    if (hx >= 0x4195b844u) {          // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {      // |x| >= 88.72...
            if (hx > 0x7f800000u) return x + x;                 // NaN
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;  // +-inf
            if (x > o_threshold) return 1.0e30f * 1.0e30f;       // overflow to +inf
        }
        if (xsb != 0) return 1.0e-30f - 1.0f;  // x < -27 ln2: -1 (inexact)
    }
    if (hx > 0x3eb17218u) {           // |x| > 0.5 ln2: argument reduction
        if (hx < 0x3F851592u) {       // and |x| < 1.5 ln2
            if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else          { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));  // truncating conversion
            t = (float)k;
            hi = x - t * ln2_hi;      // t*ln2_hi is exact here
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {    // |x| < 2^-25
        t = 1.0e30f + x;
        return x - (t - (1.0e30f + x));
    } else {
        k = 0;
    }

    const float hfx = 0.5f * x;
    const float hxs = x * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return 1.0f + 2.0f * (x - e);
    }
    float y;
    if (k <= -2 || k > 56) {          // exp(x) - 1 = 2^k (1 - (e - x)) - 1
        y = 1.0f - (e - x);
        y = bitsf(fbits(y) + ((uint32_t)k << 23));
        return y - 1.0f;
    }
    if (k < 23) {
        t = bitsf(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
        y = t - (e - x);
        y = bitsf(fbits(y) + ((uint32_t)k << 23));
    } else {
        t = bitsf((uint32_t)(0x7f - k) << 23);        // 2^-k
        y = x - (e + t);
        y += 1.0f;
        y = bitsf(fbits(y) + ((uint32_t)k << 23));
    }
    return y;
}

// n / d rounded to nearest. The device forms it from the hardware reciprocal
// and one FMA correction (q0 = n·r, q = q0 + (n − d·q0)·r), 4 instructions
// against ~10 for the IEEE sequence; for the operands glibc_tanhf divides
// here (normal numerators and denominators, normal quotients) it returns the
// IEEE quotient for every f32 input of the kernels that use it (tested on the
// GPU over all 2^32 GELU inputs and every half-precision GELU input). The host
// build divides.
__host__ __device__ inline float div_tanh(float n, float d) {
#if defined(__HIP_DEVICE_COMPILE__)
    const float r = __builtin_amdgcn_rcpf(d);
    const float q0 = n * r;
    return __builtin_fmaf(__builtin_fmaf(-d, q0, n), r, q0);
#else
    return n / d;
#endif
}

// fdlibm tanhf, written for lanes that take different branches. fdlibm
// computes, for 2^-55 <= |x| < 22,
//   |x| >= 1:  t = expm1f(2|x|),  z = 1 - 2/(t + 2)
//   |x| <  1:  t = expm1f(-2|x|), z = -t/(t + 2)
// and returns z with x's sign (|x| >= 22: 1 - 1e-30; |x| < 2^-55: x(1 + x);
// inf: +-1; NaN: NaN). tanhf_core returns fdlibm's value for every input but
// NaN, with one expm1f per element on the argument fdlibm would pass and one
// division for both formulas. Its expm1f is fdlibm's (glibc_expm1f above),
// reorganised for the arguments tanhf passes:
//  - |x| is clamped to 9.5: from |x| = 9.02 up, 2/(t + 2) < 2^-25 and fdlibm's
//    z rounds to exactly 1, as does 1 - 1e-30 beyond 22, so the clamped
//    evaluation gives fdlibm's result there, infinities included. expm1f's
//    argument a then lies in (-2, 19], where k <= 27;
//  - the three reductions are one formula: k = 0 and k = -1 are the general
//    hi = a - k·ln2_hi, lo = k·ln2_lo at that k (k·ln2_hi is exact; at k = 0,
//    hi = a, lo = +0, so the reduced argument is a and c = +0, as fdlibm has);
//  - every reconstruction starts from d = xr - e2 with
//    e2 = (xr·(e - c) - c) - hxs: at k = 0 (c = +0) e2 is fdlibm's
//    xr·e - hxs and its result is d; k = -1 gives 0.5·d - 0.5; for k <= -2,
//    2^k·(1 + d) - 1, and for k >= 2, 2^k·((1 - 2^-k) + d), fdlibm's
//    1 - (e - x) and t - (e - x) with e - x = -d exactly. fdlibm's k >= 23
//    form, (x - (e + 2^-k)) + 1, rounds differently from the k < 23 one, but
//    the two give the same tanhf for every input (for |x| >= 7.97, where
//    k >= 23, 2/(t + 2) <= 2^-21 and a last-place change in t does not move
//    1 - 2/(t + 2); checked exhaustively);
//  - |a| < 2^-25, where fdlibm returns a, is the k = 0 formula: d rounds to a;
//    so is |x| < 2^-55, where the quotient 2|x| / 2 is |x| exactly.
// Every operation is fdlibm's, in its order, rounded on its own; z >= +0, so
// x's sign is ORed in.
__host__ __device__ inline float tanhf_core(float x) {
    const float ln2_hi = 6.9313812256e-01f;  // 0x3f317180
    const float ln2_lo = 9.0580006145e-06f;  // 0x3717f7d1
    const float invln2 = 1.4426950216e+00f;  // 0x3fb8aa3b
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    const uint32_t jx = fbits(x);
    const uint32_t ix = jx & 0x7fffffffu;
    const bool big = ix >= 0x3f800000u;                          // |x| >= 1
    const float ax = bitsf(ix < 0x41180000u ? ix : 0x41180000u);  // |x|, at most 9.5
    const float a2 = 2.0f * ax;                                  // |a| (exact)
    const float a = big ? a2 : -a2;                              // expm1f's argument
    const uint32_t ha = fbits(a2);
    // k: 0 up to 0.5 ln2, else fdlibm's rounding of a / ln2 (truncating
    // conversion). Below 1.5 ln2, where fdlibm sets k = -1 without it, the
    // rounding gives -1 as well (a < 0 there: a positive argument is >= 2).
    int32_t k = (int32_t)(invln2 * a + (big ? 0.5f : -0.5f));
    if (ha <= 0x3eb17218u) k = 0;
    const float tk = (float)k;
    const float hi = a - tk * ln2_hi;
    const float lo = tk * ln2_lo;
    const float xr = hi - lo;
    const float c = (hi - xr) - lo;
    const float hfx = 0.5f * xr;
    const float hxs = xr * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    const float t3 = 3.0f - r1 * hfx;
    const float e = hxs * div_tanh(r1 - t3, 6.0f - xr * t3);
    const float e2 = (xr * (e - c) - c) - hxs;
    const float d = xr - e2;
    const float tt = k >= 2 ? bitsf(0x3f800000u - (0x1000000u >> (k & 31))) : 1.0f;  // 1 - 2^-k, or 1
    const float w = bitsf(fbits(tt + d) + ((uint32_t)k << 23));                        // scaled by 2^k
    const float em1 = k == 0 ? d : (k == -1 ? 0.5f * d - 0.5f : (k < 0 ? w - 1.0f : w));
    // tanh from expm1
    const float q = div_tanh(big ? 2.0f : -em1, em1 + 2.0f);
    const float z = big ? 1.0f - q : q;
    return bitsf(fbits(z) | (jx & 0x80000000u));
}

// glibc's tanhf for every f32 input: NaN gives a quiet NaN (fdlibm's x + x).
__host__ __device__ inline float glibc_tanhf(float x) {
    const float r = tanhf_core(x);
    return (fbits(x) & 0x7fffffffu) > 0x7f800000u ? x + x : r;
}

// GELU, tanh form, in the reference's operation order (elementwise.rs:120-127):
//   inner = 0.797_884_56 * (v + 0.044_715 * v * v * v);  y = 0.5 * v * (1 + tanh(inner))
// inner is NaN only for a NaN v (a finite or infinite v gives a finite or
// same-signed infinite inner), and then y is NaN whatever tanh returns, so
// tanh's NaN case is not needed here.
__host__ __device__ inline float gelu_tanh_ref_order(float v) {
    const float S = 0.79788456f, C = 0.044715f;
    const float inner = S * (v + C * v * v * v);
    return 0.5f * v * (1.0f + tanhf_core(inner));
}

}  // namespace sph
