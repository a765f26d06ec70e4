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
// inf: +-1; NaN: NaN). Here one expm1f runs per element, on the argument fdlibm
// would pass, and one division serves both formulas. The expm1f is fdlibm's
// (glibc_expm1f above) for the arguments tanhf passes, |a| in [2^-54, 44):
//  - its three reductions are one formula: k = 0 and k = -1 are the general
//    hi = a - k·ln2_hi, lo = k·ln2_lo at that k (k·ln2_hi is exact; at k = 0,
//    hi = a, lo = +0, so the reduced argument is a and c = +0, as fdlibm has);
//  - its reconstruction cases that these arguments reach (k = 0, -1, <= -2 or
//    > 56, < 23, else) are all evaluated and the one fdlibm takes is selected;
//  - |a| < 2^-25 returns a, as fdlibm's 1e30-trick does.
// Every operation is fdlibm's, in its order, rounded on its own, so the result
// equals glibc_tanhf's (checked against the host libm over all 2^32 inputs).
// Lanes whose result comes from a special case still run the main formula on
// a clamped argument (no out-of-range float-to-int conversion); that value is
// discarded.
__host__ __device__ inline float glibc_tanhf(float x) {
    const float ln2_hi = 6.9313812256e-01f;  // 0x3f317180
    const float ln2_lo = 9.0580006145e-06f;  // 0x3717f7d1
    const float invln2 = 1.4426950216e+00f;  // 0x3fb8aa3b
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    const uint32_t jx = fbits(x);
    const uint32_t ix = jx & 0x7fffffffu;
    const bool big = ix >= 0x3f800000u;                     // |x| >= 1
    const float ax = bitsf(ix < 0x41b00000u ? ix : 0x41a80000u);  // |x|, or 21 off the main range
    const float a = big ? 2.0f * ax : -2.0f * ax;           // expm1f's argument (exact)
    const uint32_t ha = fbits(a) & 0x7fffffffu;

    // expm1f(a)
    // A positive argument is >= 2 (|x| >= 1), past 1.5 ln2, so fdlibm's k = 1
    // case never arises here: k is -1 below 1.5 ln2, else the general k.
    int32_t k = 0;
    if (ha > 0x3eb17218u)                                   // |a| > 0.5 ln2
        k = ha < 0x3F851592u ? -1                           // |a| < 1.5 ln2 (a < 0 here)
                             : (int32_t)(invln2 * a + (big ? 0.5f : -0.5f));  // truncating conversion
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
    const float y0 = xr - (xr * e - hxs);                   // k == 0
    const float e2 = (xr * (e - c) - c) - hxs;
    const float ym1 = 0.5f * (xr - e2) - 0.5f;              // k == -1
    const uint32_t kexp = (uint32_t)k << 23;                // k added to an exponent field
    const float ya = bitsf(fbits(1.0f - (e2 - xr)) + kexp) - 1.0f;  // k <= -2 or k > 56
    const int ks = k < 0 ? 0 : (k > 31 ? 31 : k);          // shift count in range (used for 2 <= k < 23)
    const float yb = bitsf(fbits(bitsf(0x3f800000u - (0x1000000u >> ks)) - (e2 - xr)) + kexp);  // k < 23
    const float yc = bitsf(fbits((xr - (e2 + bitsf((uint32_t)(0x7f - k) << 23))) + 1.0f) + kexp);  // else
    float em1 = k == 0 ? y0 : (k == -1 ? ym1 : ((k <= -2 || k > 56) ? ya : (k < 23 ? yb : yc)));
    if (ha < 0x33000000u) em1 = a;                          // |a| < 2^-25

    // tanh from expm1
    const float q = div_tanh(big ? 2.0f : -em1, em1 + 2.0f);
    const float z = big ? 1.0f - q : q;
    float r = (jx >> 31) ? -z : z;
    if (ix >= 0x41b00000u) r = (jx >> 31) ? -(1.0f - 1.0e-30f) : 1.0f - 1.0e-30f;  // |x| >= 22
    if (ix < 0x24000000u) r = x * (1.0f + x);               // |x| < 2^-55 (and +-0)
    // fdlibm returns 1/x -+ 1: +-1 at +-inf, a NaN for a NaN (written without
    // the division, which would otherwise run on every lane).
    if (ix == 0x7f800000u) r = (jx >> 31) ? -1.0f : 1.0f;
    if (ix > 0x7f800000u) r = x + x;
    return r;
}

// GELU, tanh form, in the reference's operation order (elementwise.rs:120-127):
//   inner = 0.797_884_56 * (v + 0.044_715 * v * v * v);  y = 0.5 * v * (1 + tanh(inner))
__host__ __device__ inline float gelu_tanh_ref_order(float v) {
    const float S = 0.79788456f, C = 0.044715f;
    const float inner = S * (v + C * v * v * v);
    return 0.5f * v * (1.0f + glibc_tanhf(inner));
}

}  // namespace sph
