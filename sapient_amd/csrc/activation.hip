// activation.hip — element-wise add / mul / SiLU / SwiGLU / GELU (tanh and erf
// forms) and the last-dimension bias add, for gfx950.
//
// Reference math (crates/sapient-backends/cpu/src/kernels/elementwise.rs):
//   add  a + b                        (:61-63, broadcast rule of binary_f32 :27-57)
//   mul  a * b                        (:67-69)
//   silu v / (1 + exp(-v))            (:141-143)
//   swiglu = silu(gate) * up          (llama.rs:531-532; wgpu analog elementwise.wgsl op1)
//   gelu 0.5 v (1 + tanh(0.79788456 (v + 0.044715 v v v)))   (:120-127)
//   gelu_erf 0.5 v (1 + erf_approx(v / √2))                  (:135-138, :163-174)
//   add_bias y[i] + bias[i % n]        (crates/sapient-models/src/forward/common.rs:556-569)
//
// Design: all streams are HBM-bound. Each thread moves 16-byte vectors, two
// in flight per operand, non-temporal (every byte is touched once); the grid
// is sized so each thread makes about one trip (up to 64K blocks) — measured
// on MI355X, a near-flat grid streams faster than a grid-stride loop over few
// blocks (SwiGLU f16: 125 → 114 µs).
//  - SiLU / SwiGLU return the reference's bits. f32 evaluates the reference's
//    expression (glibc's expf restated, see glibc_expf.h, then the IEEE
//    division) on every element: ~45 VALU ops, within the budget of 8-12
//    bytes per element. Half types (4-6 bytes per element) would be
//    VALU-bound that way, so they evaluate a fast SiLU (hardware exp2 /
//    reciprocal, ≤ 5 ulp — measured over every f32 input it serves) and run
//    the exact expression only where that error could change the rounding to
//    the half type (silu_certified).
//  - GELU: the reference's 1 + tanh(z) cancels for z < -3, so its result there
//    is glibc's rounding of tanh; only glibc's own algorithm reproduces it (see
//    glibc_tanhf.h). For f16 / bf16 inputs the op is a function of 16 bits, so
//    GELU is tabulated once per device — every input with |v| < 16 evaluated
//    on the GPU with that algorithm; outside that band the result is exactly
//    v, -0 or NaN — and each launch stages the 76 KiB table in LDS (two
//    resident blocks per CU in gfx950's 160 KiB) and streams the tensor through it:
//    bit-exact and bandwidth-bound. f32 inputs evaluate the algorithm per
//    element (VALU-bound).
//  - erf-GELU takes the same two routes: its erf_approx multiplies by glibc's
//    expf(-x²), restated in glibc_expf.h (double-precision evaluation with a
//    32-entry table of 2^(i/32), which each block stages in LDS). Outside
//    |v| < 16 expf(-x²) underflows to 0, so the band and the outside rule are
//    the ones of the tanh form.
//  - Bias add: a block owns a tile of up to 256 16-byte column vectors over
//    two rows; each thread loads its bias vector once and adds it to both.
#include <mutex>
#include <type_traits>

#include "glibc_expf.h"
#include "glibc_tanhf.h"
#include "sph_common.h"

namespace sph {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 2;       // vectors in flight per operand per thread
constexpr int64_t kMaxGrid = 65536;  // ~one loop trip per thread at the configuration sizes
// Launches of up to 2^20 16-byte vectors take one vector per thread (a single trip, each thread's
// chain as short as it can be). Per launch, back to back on MI355X, against two vectors per thread:
// SwiGLU 64 x 14336 f32 3.99 -> 3.03 µs, f16 5.42 -> 3.53; 512 x 4864 f32 7.10 -> 6.46, f16 7.08 ->
// 5.16; 512 x 14336 f16 11.7 -> 11.2; GELU-tanh f32 512 x 4864 6.88 -> 6.60, but at 512 x 14336 f32
// (1.8 M vectors) 14.2 -> 16.1, and at larger launches both shapes run alike.
constexpr int64_t kFewVecs = int64_t(1) << 20;

// Launches of up to 2^18 elements (decode steps, small prefill chunks) take one element per thread
// instead, for every op whose per-element work is long (half-precision I/O, GELU) and for f32 from
// 2048 elements on: a thread's chain is then one element's, and half-precision GELU reads its
// table from cache rather than staging it per block. Per launch (replayed graph, back to back) on
// MI355X, against the vector shapes: SwiGLU and SiLU f16 / bf16 -21 to -36 % (SwiGLU 1 x 4864 f16
// 2.58 -> 1.83 µs), GELU-tanh f16 / bf16 -16 to -40 % (1 x 10240 f16 2.90 -> 1.79 µs), GELU-tanh
// f32 -16 to -23 %, SwiGLU f32 -4 to -6 % from 4864 elements (1.92 -> 1.82 µs); below 2048 f32
// elements the light ops measured level or 0.3 % slower, and at 2^19 elements both shapes ran
// alike (bf16 GELU 5.9 % slower one element per thread), hence the bounds. Results are the same
// bits either way.
constexpr int64_t kFewElems = int64_t(1) << 18;
constexpr int64_t kFewF32LightMin = 2048;

enum Op { OP_ADD = 0, OP_MUL = 1, OP_SILU = 2, OP_SWIGLU = 3, OP_GELU = 4, OP_GELU_ERF = 5 };

// 2^(i/32) for the expf restatement, staged per block into LDS by the kernels that need it.
__constant__ Exp2fTable kExp2f = exp2f_table();
enum Bcast { B_NONE = 0, B_SCALAR_B = 1, B_SCALAR_A = 2 };

// Fast SiLU for g >= -80: exp(-g) from the hardware exp2 on a split-precision
// argument, 1 / (1 + e) from the hardware reciprocal, ~12 VALU ops. Above 64,
// exp(-g) < 2^-92, so 1 + e rounds to 1 and the reference returns g itself.
__device__ __forceinline__ float silu_f(float g) {
    if (g > 64.0f) return g;
    const float kL2eHi = 1.44269502162933349609375f;  // f32(log2 e)
    const float kL2eLo = 1.925963033500011e-08f;      // log2 e - kL2eHi
    const float kLn2 = 0.693147180559945309f;
    const float ng = -g;
    const float p = ng * kL2eHi;
    const float perr = __builtin_fmaf(ng, kL2eHi, -p) + ng * kL2eLo;  // -g·log2e - p
    const float e0 = __builtin_amdgcn_exp2f(p);
    const float e = __builtin_fmaf(e0, perr * kLn2, e0);            // 2^(p + perr)
    return g * __builtin_amdgcn_rcpf(1.0f + e);
}

// True when every f32 within 16 ulp of p rounds to the same T: p is far enough
// from the midpoint between two T values (a window around a midpoint never
// reaches a binade edge, so bit units are ulps). f16: the 13 bits below its
// mantissa, for |p| in [2^-14, 2^16) (normal f16 results and their overflow to
// inf); bf16: the 16 bits below its mantissa, anywhere in the finite range.
template <typename T>
__device__ __forceinline__ bool rounding_is_clear(float p) {
    const uint32_t b = __builtin_bit_cast(uint32_t, p);
    const uint32_t e = (b >> 23) & 0xFFu;
    if constexpr (std::is_same<T, f16>::value) {
        if (e < 113u || e > 142u) return false;
        const int low = (int)(b & 0x1FFFu) - 0x1000;
        return low > 16 || low < -16;
    } else {
        if (e == 0xFFu || e < 2u) return false;
        const int low = (int)(b & 0xFFFFu) - 0x8000;
        return low > 16 || low < -16;
    }
}

// SiLU (times u for SwiGLU) whose rounding to the half type T equals the
// reference's: the fast silu_f is certified where it decides the result. Over
// every f32 g in [-80, 64] silu_f lies within 5 ulp of the exact
// silu_ref_order (measured on MI355X over all 2^31 such inputs). In ulps of
// the product that is < 10 ulp (ulp(s)·|u| < 2 ulp(s·u)), and the roundings
// RN(s·u), RN(s'·u) add one more, so the exact result lies within 11 ulp of the
// fast p. When every f32 within 16 ulp of p rounds to the same T value,
// rounding being monotonic, so does the exact result. Otherwise (about 0.4 %
// of elements), outside the measured domain, for non-finite values and for
// results outside the ranges rounding_is_clear covers, the exact expression
// runs inline: it touches only registers and the LDS copy of the 2^(i/32)
// table, so its rare divergent executions cost ~1 % (measured: fast-only
// 112 µs, certified 113 µs on f16 SwiGLU [8192, 14336]; a table load from
// global memory in the same branch stalls the wave on its stream traffic,
// 136 µs).
template <typename T, bool MUL>
__device__ __forceinline__ float silu_certified(float g, float u, const uint64_t* exp_tab) {
    const float s = silu_f(g);
    const float p = MUL ? s * u : s;
    if (g >= -80.0f && rounding_is_clear<T>(p)) return p;
    const float x = silu_ref_order(g, exp_tab);
    return MUL ? x * u : x;
}

// T: the storage type. SiLU / SwiGLU give the reference's bits: f32 evaluates
// the reference's expression exactly (glibc's expf restated, IEEE division —
// within the bandwidth budget of 8-12 bytes per element); half types take the
// certified fast path (4-6 bytes per element leave no room for the exact
// expression on every element: f16 SwiGLU 149 µs instead of 113).
template <int OP, typename T>
__device__ __forceinline__ float apply_op(float a, float b, const uint64_t* exp_tab) {
    constexpr bool kExact = sizeof(T) == 4;
    if constexpr (OP == OP_ADD) return a + b;
    if constexpr (OP == OP_MUL) return a * b;
    if constexpr (OP == OP_SILU) {
        if constexpr (kExact) return silu_ref_order(a, exp_tab);
        else return silu_certified<T, false>(a, 0.0f, exp_tab);
    }
    if constexpr (OP == OP_SWIGLU) {
        if constexpr (kExact) return silu_ref_order(a, exp_tab) * b;
        else return silu_certified<T, true>(a, b, exp_tab);
    }
    if constexpr (OP == OP_GELU) return gelu_tanh_ref_order(a);
    if constexpr (OP == OP_GELU_ERF) return gelu_erf_ref_order(a, exp_tab);
    return 0.0f;
}

template <int OP, typename T> constexpr bool needs_exp_table() {
    return OP == OP_GELU_ERF || OP == OP_SILU || OP == OP_SWIGLU;
}

// Copy the 2^(i/32) table into LDS (block-wide; call before any use).
__device__ __forceinline__ void stage_exp_table(uint64_t* tab) {
    if (threadIdx.x < 32) tab[threadIdx.x] = kExp2f.tab[threadIdx.x];
    __syncthreads();
}

template <int OP> constexpr bool binary_op() { return OP == OP_ADD || OP == OP_MUL || OP == OP_SWIGLU; }

// Vector path: nvec 16-byte vectors of T; a, b, out all 16-byte aligned.
// B_SCALAR_B / B_SCALAR_A read element 0 of the broadcast operand. `out` may
// alias a full-length input: each element is read before it is written, by
// the same thread.
template <typename T, int OP, int BC, int U = kUnroll>
__global__ __launch_bounds__(kThreads) void ew_vec(const T* a, const T* b, T* out, int64_t nvec) {
    constexpr int E = vec16<T>::n;
    __shared__ uint64_t exp_tab[needs_exp_table<OP, T>() ? 32 : 1];
    if constexpr (needs_exp_table<OP, T>()) stage_exp_table(exp_tab);
    float sa = 0.0f, sb = 0.0f;
    if constexpr (BC == B_SCALAR_A) sa = widen(a[0]);
    if constexpr (BC == B_SCALAR_B) sb = widen(b[0]);
    const int64_t stride = (int64_t)gridDim.x * kThreads * U;
    for (int64_t base = (int64_t)blockIdx.x * kThreads * U + threadIdx.x; base < nvec; base += stride) {
        float va[U][E], vb[U][E];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = base + (int64_t)u * kThreads;
            if (i < nvec) {
                if constexpr (BC != B_SCALAR_A) load_f32<T, E, true>(a + i * E, va[u]);
                if constexpr (binary_op<OP>() && BC != B_SCALAR_B) load_f32<T, E, true>(b + i * E, vb[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = base + (int64_t)u * kThreads;
            if (i < nvec) {
                float o[E];
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const float x = BC == B_SCALAR_A ? sa : va[u][e];
                    const float y = BC == B_SCALAR_B ? sb : vb[u][e];
                    o[e] = apply_op<OP, T>(x, y, exp_tab);
                }
                store_f32<T, E, true>(out + i * E, o);
            }
        }
    }
}

// Scalar path for misaligned pointers and the tail past the last full vector.
template <typename T, int OP, int BC>
__global__ __launch_bounds__(kThreads) void ew_scalar(const T* a, const T* b, T* out, int64_t begin,
                                                      int64_t end) {
    __shared__ uint64_t exp_tab[needs_exp_table<OP, T>() ? 32 : 1];
    if constexpr (needs_exp_table<OP, T>()) stage_exp_table(exp_tab);
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < end; i += stride) {
        const float x = widen(a[BC == B_SCALAR_A ? 0 : i]);
        const float y = binary_op<OP>() ? widen(b[BC == B_SCALAR_B ? 0 : i]) : 0.0f;
        out[i] = narrow<T>(apply_op<OP, T>(x, y, exp_tab));
    }
}

inline unsigned grid_for(int64_t items, int64_t per_block, int64_t cap) {
    int64_t g = (items + per_block - 1) / per_block;
    if (g < 1) g = 1;
    return (unsigned)(g < cap ? g : cap);
}

template <typename T, int OP, int BC>
int launch_ew(const void* a, const void* b, void* out, int64_t n, hipStream_t stream) {
    if (n == 0) return SPH_OK;
    constexpr int E = vec16<T>::n;
    const T* ap = static_cast<const T*>(a);
    const T* bp = static_cast<const T*>(b);
    T* op = static_cast<T*>(out);
    constexpr bool kLongChain = sizeof(T) == 2 || OP == OP_GELU || OP == OP_GELU_ERF;
    if (n <= kFewElems && (kLongChain || n >= kFewF32LightMin))
        return launch(ew_scalar<T, OP, BC>, grid_for(n, kThreads, 4096), kThreads, stream, ap, bp, op, (int64_t)0, n);
    const bool vec_ok = aligned(out, 16) && (BC == B_SCALAR_A || aligned(a, 16)) &&
                        (!binary_op<OP>() || BC == B_SCALAR_B || aligned(b, 16));
    int64_t done = 0;
    if (vec_ok) {
        const int64_t nvec = n / E;
        if (nvec > 0 && nvec <= kFewVecs) {
            // A small or mid-size launch (a decode step, a prefill chunk): one vector per thread.
            const int st = launch(ew_vec<T, OP, BC, 1>, grid_for(nvec, (int64_t)kThreads, kMaxGrid), kThreads, stream,
                                  ap, bp, op, nvec);
            if (st != SPH_OK) return st;
        } else if (nvec > 0) {
            const int st = launch(ew_vec<T, OP, BC>, grid_for(nvec, (int64_t)kThreads * kUnroll, kMaxGrid), kThreads,
                                  stream, ap, bp, op, nvec);
            if (st != SPH_OK) return st;
        }
        done = nvec * E;
    }
    if (done < n) {
        const int st = launch(ew_scalar<T, OP, BC>, grid_for(n - done, kThreads, 4096), kThreads, stream, ap, bp, op,
                              done, n);
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

template <int OP>
int dispatch_unary(const void* x, void* out, int dt, int64_t n, hipStream_t stream) {
    if (n < 0) return SPH_EINVAL;
    if (n > 0 && (x == nullptr || out == nullptr)) return SPH_EINVAL;
    return with_float_type(dt, [&](auto t) -> int {
        using T = decltype(t);
        return launch_ew<T, OP, B_NONE>(x, nullptr, out, n, stream);
    });
}

template <int OP>
int dispatch_binary(const void* a, int64_t na, const void* b, int64_t nb, void* out, int dt, hipStream_t stream) {
    if (na < 0 || nb < 0) return SPH_EINVAL;
    if (a == nullptr || b == nullptr || out == nullptr) {
        if (na == 0 && nb == 0) return SPH_OK;
        return SPH_EINVAL;
    }
    return with_float_type(dt, [&](auto t) -> int {
        using T = decltype(t);
        if (na == nb) return launch_ew<T, OP, B_NONE>(a, b, out, na, stream);
        if (nb == 1) return launch_ew<T, OP, B_SCALAR_B>(a, b, out, na, stream);
        if (na == 1) return launch_ew<T, OP, B_SCALAR_A>(a, b, out, nb, stream);
        return SPH_EINVAL;  // the reference's ShapeMismatch
    });
}

// ─────────────────────────── GELU lookup tables ───────────────────────────
// For |v| >= 16 GELU is exact without a table: tanh(z) rounds to ±1, so the
// reference returns v itself for v >= 16 (and +inf), -0 for v <= -16, and
// NaN for -inf (-inf · 0) and NaN. The table therefore holds only |v| < 16:
// the 16-bit patterns below kLimit, for both signs — 76 KiB for f16 (68 KiB
// for bf16), which lets two 1024-thread blocks share a CU's 160 KiB of LDS.
template <typename T> struct gelu_band;
template <> struct gelu_band<f16> {   // 16.0 = 0x4C00; +inf 0x7C00; quiet-NaN bit 0x0200
    static constexpr uint32_t kLimit = 0x4C00u, kInf = 0x7C00u, kQuiet = 0x0200u;
};
template <> struct gelu_band<bf16> {  // 16.0 = 0x4180; +inf 0x7F80; quiet-NaN bit 0x0040
    static constexpr uint32_t kLimit = 0x4180u, kInf = 0x7F80u, kQuiet = 0x0040u;
};
constexpr uint32_t kLutEntries = 2 * gelu_band<f16>::kLimit;  // the larger of the two

// Table slot of a pattern inside the band: positives first, then negatives.
template <typename T>
__device__ __forceinline__ uint32_t gelu_slot(uint32_t h) {
    return (h & 0x8000u) ? gelu_band<T>::kLimit + (h & 0x7FFFu) : h;
}

// Result for a pattern outside the band (|v| >= 16, inf, NaN).
template <typename T>
__device__ __forceinline__ uint32_t gelu_outside(uint32_t h) {
    constexpr uint32_t inf = gelu_band<T>::kInf, quiet = gelu_band<T>::kQuiet;
    const bool neg = (h & 0x8000u) != 0;
    const uint32_t mag = h & 0x7FFFu;
    if (mag > inf) return h | quiet;                  // NaN stays NaN (quiet)
    if (!neg) return h;                               // v >= 16 and +inf: v
    if (mag == inf) return 0x8000u | inf | quiet;     // -inf: -inf * 0 = NaN
    return 0x8000u;                                   // v <= -16: -0
}

// Tables by index: form * 2 + type, form 0 = tanh, 1 = erf; type 0 = f16, 1 = bf16.
constexpr int kLutTables = 4;
__device__ __align__(16) uint16_t gelu_lut[kLutTables][kLutEntries];

template <typename T>
__global__ __launch_bounds__(kThreads) void gelu_lut_build(int which) {
    __shared__ uint64_t exp_tab[32];
    stage_exp_table(exp_tab);
    const uint32_t slot = blockIdx.x * kThreads + threadIdx.x;
    constexpr uint32_t L = gelu_band<T>::kLimit;
    if (slot >= 2 * L) return;
    const uint32_t h = slot < L ? slot : 0x8000u | (slot - L);
    const float v = widen(T{(uint16_t)h});
    const float g = which < 2 ? gelu_tanh_ref_order(v) : gelu_erf_ref_order(v, exp_tab);
    gelu_lut[which][slot] = narrow<T>(g).bits;
}

constexpr int kLutThreads = 512;
constexpr int kLutBatch = 2;  // 16-byte vectors per thread per trip

template <typename T>
__device__ __forceinline__ uint32_t gelu_lookup(const uint16_t* tab, uint32_t h) {
    return (h & 0x7FFFu) < gelu_band<T>::kLimit ? (uint32_t)tab[gelu_slot<T>(h)] : gelu_outside<T>(h);
}

// Two 512-thread blocks per CU, both resident (LDS-bound), each staging the
// band table in LDS once and then streaming 16-byte vectors, grid-stride, U
// per thread per trip. Measured on MI355X at [8192, 10240] f16, round-robin
// with a 16-byte copy of the same bytes (53.9 µs in this loop shape, 53.1 as
// a flat grid): U = 2 56.8 µs, U = 3 58.6, U = 4 59.4, U = 1 62.8; four
// blocks per CU (the table staged twice per slot) 59.4 at U = 2; the first
// trip's loads issued before the table is staged: no change. Earlier:
// 1024-thread blocks or the next trip's loads issued ahead (software
// pipelining) 63-65.
template <typename T, int U>
__global__ __launch_bounds__(kLutThreads) void gelu_lut_apply(const uint16_t* in, uint16_t* out, int64_t nvec, int which) {
    __shared__ __align__(16) uint16_t tab[kLutEntries];
    {
        // The table is copied into LDS with gfx950's direct-to-LDS 16-byte
        // loads (global_load_lds_dwordx4: lane l of a wave writes the 16 bytes
        // at the wave's LDS base + 16 l, no register round trip), all of a
        // thread's chunks requested before the wait: one L2 round trip per block
        // (a load-wait-store loop through registers serialised ten of them; the
        // register-staged form of the same loop measured 0.2-0.4 us slower).
        constexpr int nq = (int)(2 * gelu_band<T>::kLimit * 2 / 16);  // 16-byte chunks of this type's table
        constexpr int per = (nq + kLutThreads - 1) / kLutThreads;
        // A wave loads 64 chunks from its base, and only waves whose base is below nq load.
        static_assert((nq + 63) / 64 * 64 <= (int)(kLutEntries * 2 / 16), "a wave's chunks stay inside tab");
        const u32x4* src = reinterpret_cast<const u32x4*>(gelu_lut[which]);
        const int wv = (int)threadIdx.x / 64;
#pragma unroll
        for (int i = 0; i < per; ++i) {
            const int base = i * kLutThreads + wv * 64;  // this wave's first chunk (wave-uniform)
            if (base < nq) {
                // Lanes past the table's end reload its last chunk into tab's
                // spare slots (in bounds: see the static_assert).
                const int k = (int)threadIdx.x + i * kLutThreads;
                __builtin_amdgcn_global_load_lds(src + (k < nq ? k : nq - 1), reinterpret_cast<u32x4*>(tab) + base,
                                                 16, 0, 0);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    const u32x4* vin = reinterpret_cast<const u32x4*>(in);
    u32x4* vout = reinterpret_cast<u32x4*>(out);
    const int64_t stride = (int64_t)gridDim.x * kLutThreads * U;
    for (int64_t base = (int64_t)blockIdx.x * kLutThreads * U + threadIdx.x; base < nvec; base += stride) {
        u32x4 q[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = base + (int64_t)u * kLutThreads;
            if (i < nvec) q[u] = vload<true>(vin + i);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = base + (int64_t)u * kLutThreads;
            if (i < nvec) {
                u32x4 r;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const uint32_t w = q[u][c];
                    r[c] = gelu_lookup<T>(tab, w & 0xFFFFu) | (gelu_lookup<T>(tab, w >> 16) << 16);
                }
                vstore<true>(vout + i, r);
            }
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void gelu_lut_apply_scalar(const uint16_t* in, uint16_t* out, int64_t begin,
                                                                  int64_t end, int which) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < end; i += stride)
        out[i] = (uint16_t)gelu_lookup<T>(gelu_lut[which], in[i]);
}

constexpr int kMaxDevices = 64;
std::mutex g_init_mu;
bool g_lut_ready[kMaxDevices];
int g_num_cus[kMaxDevices];

// Build the four tables on `stream` once per device and wait for them.
int ensure_device_ready(hipStream_t stream, int* cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return SPH_ENODEV;
    std::lock_guard<std::mutex> lock(g_init_mu);
    if (!g_lut_ready[dev]) {
        // The build waits for its kernels: under stream capture they would be
        // recorded instead of run and the wait would invalidate the capture.
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return SPH_EHIP;
        if (cap != hipStreamCaptureStatusNone) return SPH_ESTATE;
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            return SPH_ENODEV;
        g_num_cus[dev] = n;
        const dim3 grid((kLutEntries + kThreads - 1) / kThreads);
        for (int form = 0; form < 2; ++form) {
            if (launch(gelu_lut_build<f16>, grid, kThreads, stream, form * 2) != SPH_OK) return SPH_EHIP;
            if (launch(gelu_lut_build<bf16>, grid, kThreads, stream, form * 2 + 1) != SPH_OK) return SPH_EHIP;
        }
        if (hipStreamSynchronize(stream) != hipSuccess) return SPH_EHIP;
        g_lut_ready[dev] = true;
    }
    if (cus) *cus = g_num_cus[dev];
    return SPH_OK;
}

template <typename T>
int gelu_half(const uint16_t* x, uint16_t* out, int which, int64_t n, hipStream_t stream) {
    int cus = 0;
    int st = ensure_device_ready(stream, &cus);
    if (st != SPH_OK) return st;
    if (n <= kFewElems)  // one element per thread, the table read from cache (see kFewElems)
        return launch(gelu_lut_apply_scalar<T>, grid_for(n, kThreads, 4096), kThreads, stream, x, out, (int64_t)0, n,
                      which);
    int64_t done = 0;
    if (aligned(x, 16) && aligned(out, 16)) {
        const int64_t nvec = n / 8;
        if (nvec > 0) {
            st = launch(gelu_lut_apply<T, kLutBatch>, grid_for(nvec, (int64_t)kLutThreads * kLutBatch, 2 * cus),
                        kLutThreads, stream, x, out, nvec, which);
            if (st != SPH_OK) return st;
        }
        done = nvec * 8;
    }
    if (done < n) {
        st = launch(gelu_lut_apply_scalar<T>, grid_for(n - done, kThreads, 4096), kThreads, stream, x, out, done, n,
                    which);
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

// GELU of either form: half types through the tables, f32 per element.
template <int OP>
int gelu_any(const void* x, void* out, int dtype, int64_t n, hipStream_t s) {
    if (n < 0) return SPH_EINVAL;
    if (n > 0 && (x == nullptr || out == nullptr)) return SPH_EINVAL;
    if (n == 0) return is_float_dtype(dtype) ? SPH_OK : SPH_EINVAL;
    const int form = OP == OP_GELU ? 0 : 1;
    if (dtype == SPH_F16)
        return gelu_half<f16>(static_cast<const uint16_t*>(x), static_cast<uint16_t*>(out), form * 2, n, s);
    if (dtype == SPH_BF16)
        return gelu_half<bf16>(static_cast<const uint16_t*>(x), static_cast<uint16_t*>(out), form * 2 + 1, n, s);
    return dispatch_unary<OP>(x, out, dtype, n, s);
}

// ───────────────────────────── bias add ─────────────────────────────
// Two rows per block, both in flight: measured on MI355X at 16384 x 4096 f32
// this runs at the speed of a plain two-stream add (16 rows per block: -15 %).
constexpr int kBiasRowsPerBlock = 2;

// Block b covers column tile b % ntiles (up to 256 16-byte vectors of a row)
// over rows [(b / ntiles) · R, + R). A thread keeps its bias vector in
// registers and streams y down the rows, RU rows in flight.
template <typename T, typename TB>
__global__ __launch_bounds__(kThreads) void bias_rows_vec(const T* y, const TB* bias, T* out, int64_t rows, int nvr,
                                                         int ntiles, int tile) {
    constexpr int E = vec16<T>::n;
    constexpr int RU = 2;
    const int t = (int)(blockIdx.x % (unsigned)ntiles);
    const int64_t r0 = (int64_t)(blockIdx.x / (unsigned)ntiles) * kBiasRowsPerBlock;
    const int v = t * tile + (int)threadIdx.x;
    if ((int)threadIdx.x >= tile || v >= nvr) return;
    float bv[E];
    load_f32<TB, E>(bias + (size_t)v * E, bv);
    const int64_t r_end = r0 + kBiasRowsPerBlock < rows ? r0 + kBiasRowsPerBlock : rows;
    for (int64_t r = r0; r < r_end; r += RU) {
        float q[RU][E];
#pragma unroll
        for (int u = 0; u < RU; ++u)
            if (r + u < r_end) load_f32<T, E, true>(y + ((size_t)(r + u) * nvr + v) * E, q[u]);
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            if (r + u < r_end) {
#pragma unroll
                for (int e = 0; e < E; ++e) q[u][e] = q[u][e] + bv[e];
                store_f32<T, E, true>(out + ((size_t)(r + u) * nvr + v) * E, q[u]);
            }
        }
    }
}

// Any width / alignment: element-wise with one modulo per element.
template <typename T, typename TB>
__global__ __launch_bounds__(kThreads) void bias_scalar(const T* y, const TB* bias, T* out, int64_t total, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += stride)
        out[i] = narrow<T>(widen(y[i]) + widen(bias[i % n]));
}

template <typename T, typename TB>
int launch_bias(const void* y, const void* bias, void* out, int64_t total, int64_t n, hipStream_t stream) {
    constexpr int E = vec16<T>::n;
    const T* yp = static_cast<const T*>(y);
    const TB* bp = static_cast<const TB*>(bias);
    T* op = static_cast<T*>(out);
    const int64_t rows = total / n;
    const int64_t nvr = n / E;
    const bool vec_ok = n % E == 0 && aligned(y, 16) && aligned(out, 16) && aligned(bias, 16) &&
                        nvr <= (int64_t)1 << 24;
    if (vec_ok) {
        const int tile = nvr >= kThreads ? kThreads : (int)((nvr + 63) / 64 * 64);
        const int ntiles = (int)((nvr + tile - 1) / tile);
        const int64_t groups = (rows + kBiasRowsPerBlock - 1) / kBiasRowsPerBlock;
        // The grid is one launch: ntiles · groups < 2^32 blocks is checked here.
        if ((int64_t)ntiles * groups < ((int64_t)1 << 31)) {
            return launch(bias_rows_vec<T, TB>, dim3((unsigned)(ntiles * groups)), tile, stream, yp, bp, op, rows,
                          (int)nvr, ntiles, tile);
        }
    }
    return launch(bias_scalar<T, TB>, grid_for(total, kThreads, 65536), kThreads, stream, yp, bp, op, total, n);
}

int dispatch_bias(const void* y, const void* bias, int b_dt, void* out, int dt, int64_t total, int64_t n,
                  hipStream_t stream) {
    if (total < 0 || n < 0) return SPH_EINVAL;
    if (!is_float_dtype(dt) || !is_float_dtype(b_dt)) return SPH_EINVAL;
    if (total == 0) return SPH_OK;
    if (n == 0 || total % n != 0) return SPH_EINVAL;
    if (y == nullptr || bias == nullptr || out == nullptr) return SPH_EINVAL;
    return with_float_type(dt, [&](auto ty) -> int {
        using T = decltype(ty);
        return with_float_type(b_dt, [&](auto tb) -> int {
            using TB = decltype(tb);
            return launch_bias<T, TB>(y, bias, out, total, n, stream);
        });
    });
}

}  // namespace
}  // namespace sph

extern "C" int sph_init(void* stream) { return sph::ensure_device_ready(static_cast<hipStream_t>(stream), nullptr); }

extern "C" int sph_add(const void* a, int64_t na, const void* b, int64_t nb, void* out, int dtype, void* stream) {
    return sph::dispatch_binary<sph::OP_ADD>(a, na, b, nb, out, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int sph_mul(const void* a, int64_t na, const void* b, int64_t nb, void* out, int dtype, void* stream) {
    return sph::dispatch_binary<sph::OP_MUL>(a, na, b, nb, out, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int sph_silu(const void* x, void* out, int dtype, int64_t n, void* stream) {
    return sph::dispatch_unary<sph::OP_SILU>(x, out, dtype, n, static_cast<hipStream_t>(stream));
}

extern "C" int sph_swiglu(const void* gate, const void* up, void* out, int dtype, int64_t n, void* stream) {
    if (n < 0) return SPH_EINVAL;
    return sph::dispatch_binary<sph::OP_SWIGLU>(gate, n, up, n, out, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int sph_gelu_tanh(const void* x, void* out, int dtype, int64_t n, void* stream) {
    return sph::gelu_any<sph::OP_GELU>(x, out, dtype, n, static_cast<hipStream_t>(stream));
}

extern "C" int sph_gelu_erf(const void* x, void* out, int dtype, int64_t n, void* stream) {
    return sph::gelu_any<sph::OP_GELU_ERF>(x, out, dtype, n, static_cast<hipStream_t>(stream));
}

extern "C" int sph_add_bias(const void* y, const void* bias, int bias_dtype, void* out, int dtype, int64_t total,
                            int64_t n, void* stream) {
    return sph::dispatch_bias(y, bias, bias_dtype, out, dtype, total, n, static_cast<hipStream_t>(stream));
}
