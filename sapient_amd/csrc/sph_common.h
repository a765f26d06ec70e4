// sph_common.h — device helpers shared by the gfx950 kernels: storage types,
// exact widening / round-to-nearest-even narrowing, 16-byte vector access,
// wave64 reductions, and host-side launch plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <tuple>
#include <utility>

#include "sapient_hip.h"

namespace sph {

// ───────────────────────────── storage types ─────────────────────────────
// f16 and bf16 travel as raw 16-bit patterns; arithmetic is always f32.
struct f16 { uint16_t bits; };
struct bf16 { uint16_t bits; };
static_assert(sizeof(f16) == 2 && sizeof(bf16) == 2, "half storage must be 2 bytes");

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float widen(float v) { return v; }
__device__ __forceinline__ float widen(f16 v) {
    // v_cvt_f32_f16: exact, f16 subnormals included (f16 denormals are on by default).
    return (float)__builtin_bit_cast(_Float16, v.bits);
}
__device__ __forceinline__ float widen(bf16 v) { return __uint_as_float((uint32_t)v.bits << 16); }

template <typename T> __device__ __forceinline__ T narrow(float v);
template <> __device__ __forceinline__ float narrow<float>(float v) { return v; }
template <> __device__ __forceinline__ f16 narrow<f16>(float v) {
    // v_cvt_f16_f32 rounds to nearest-even (default MODE), keeps subnormals.
    return f16{__builtin_bit_cast(uint16_t, (_Float16)v)};
}
template <> __device__ __forceinline__ bf16 narrow<bf16>(float v) {
    // v_cvt_pk_bf16_f32 (gfx950): round to nearest-even under the default
    // MODE, subnormals kept, NaN quieted as (bits >> 16) | 0x40. Over all 2^32
    // f32 inputs on gfx950 it gives exactly the integer sequence
    // x += 0x7FFF + ((x >> 16) & 1), x >> 16, with that NaN rule.
    return bf16{__builtin_bit_cast(uint16_t, (__bf16)v)};
}
// Two values in one v_cvt_pk_bf16_f32, v0 in the low half.
__device__ __forceinline__ uint32_t narrow2_bf16(float v0, float v1) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){v0, v1}, bf16x2_t));
}
// Two values in one v_cvt_pk_f16_f32 (gfx950), v0 in the low half: the same
// bits as two v_cvt_f16_f32 (round to nearest-even under the default MODE,
// subnormals kept) for every f32 input, in one instruction instead of three.
__device__ __forceinline__ uint32_t narrow2_f16(float v0, float v1) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){v0, v1}, f16x2_t));
}

// Elements of T that fill one 16-byte access.
template <typename T> struct vec16 { static constexpr int n = 16 / (int)sizeof(T); };

// 16-byte-or-smaller vector access, optionally non-temporal (streaming data
// that is touched once: it bypasses cache residency, which measurably raises
// achieved HBM bandwidth on gfx950 for read-once / write-once streams).
template <bool NT, typename V>
__device__ __forceinline__ V vload(const V* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <bool NT, typename V>
__device__ __forceinline__ void vstore(V* p, V v) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

// Raw 32-bit words of N consecutive elements of T: N * sizeof(T) a multiple
// of 4 bytes, the address aligned to min(16, N * sizeof(T)).
template <typename T, int N> struct words_of { static constexpr int n = N * (int)sizeof(T) / 4; };

template <typename T, int N, bool NT = false>
__device__ __forceinline__ void load_words(const T* __restrict__ p, uint32_t (&raw)[words_of<T, N>::n]) {
    constexpr int bytes = N * (int)sizeof(T);
    static_assert(bytes % 4 == 0, "vector access must be whole dwords");
    if constexpr (bytes % 16 == 0) {
#pragma unroll
        for (int c = 0; c < bytes / 16; ++c) {
            u32x4 q = vload<NT>(reinterpret_cast<const u32x4*>(p) + c);
            raw[4 * c] = q.x; raw[4 * c + 1] = q.y; raw[4 * c + 2] = q.z; raw[4 * c + 3] = q.w;
        }
    } else if constexpr (bytes % 8 == 0) {
#pragma unroll
        for (int c = 0; c < bytes / 8; ++c) {
            u32x2 q = vload<NT>(reinterpret_cast<const u32x2*>(p) + c);
            raw[2 * c] = q.x; raw[2 * c + 1] = q.y;
        }
    } else {
#pragma unroll
        for (int c = 0; c < bytes / 4; ++c) raw[c] = vload<NT>(reinterpret_cast<const uint32_t*>(p) + c);
    }
}

template <typename T, int N>
__device__ __forceinline__ void words_to_f32(const uint32_t (&raw)[words_of<T, N>::n], float (&v)[N]) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = __uint_as_float(raw[i]);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            uint16_t h = (uint16_t)(raw[i / 2] >> (16 * (i & 1)));
            v[i] = widen(T{h});
        }
    }
}

template <typename T, int N>
__device__ __forceinline__ void f32_to_words(const float (&v)[N], uint32_t (&raw)[words_of<T, N>::n]) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int i = 0; i < N; ++i) raw[i] = __float_as_uint(v[i]);
    } else if constexpr (sizeof(T) == 2 && __is_same(T, bf16)) {
#pragma unroll
        for (int i = 0; i < N; i += 2) raw[i / 2] = narrow2_bf16(v[i], v[i + 1]);
    } else {
#pragma unroll
        for (int i = 0; i < N; i += 2) raw[i / 2] = narrow2_f16(v[i], v[i + 1]);
    }
}

template <typename T, int N, bool NT = false>
__device__ __forceinline__ void store_words(T* __restrict__ p, const uint32_t (&raw)[words_of<T, N>::n]) {
    constexpr int bytes = N * (int)sizeof(T);
    static_assert(bytes % 4 == 0, "vector access must be whole dwords");
    if constexpr (bytes % 16 == 0) {
#pragma unroll
        for (int c = 0; c < bytes / 16; ++c) {
            u32x4 q = {raw[4 * c], raw[4 * c + 1], raw[4 * c + 2], raw[4 * c + 3]};
            vstore<NT>(reinterpret_cast<u32x4*>(p) + c, q);
        }
    } else if constexpr (bytes % 8 == 0) {
#pragma unroll
        for (int c = 0; c < bytes / 8; ++c) {
            u32x2 q = {raw[2 * c], raw[2 * c + 1]};
            vstore<NT>(reinterpret_cast<u32x2*>(p) + c, q);
        }
    } else {
#pragma unroll
        for (int c = 0; c < bytes / 4; ++c) vstore<NT>(reinterpret_cast<uint32_t*>(p) + c, raw[c]);
    }
}

// Load N consecutive elements of T (same alignment rule) into f32 registers.
template <typename T, int N, bool NT = false>
__device__ __forceinline__ void load_f32(const T* __restrict__ p, float (&v)[N]) {
    uint32_t raw[words_of<T, N>::n];
    load_words<T, N, NT>(p, raw);
    words_to_f32<T, N>(raw, v);
}

// Store N f32 values as consecutive elements of T (same alignment rule).
template <typename T, int N, bool NT = false>
__device__ __forceinline__ void store_f32(T* __restrict__ p, const float (&v)[N]) {
    uint32_t raw[words_of<T, N>::n];
    f32_to_words<T, N>(v, raw);
    store_words<T, N, NT>(p, raw);
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the 64 lanes of a wave (all lanes active), returned to every lane.
// Within each 16-lane row four DPP steps pair lanes symmetrically (xor 1,
// xor 2, mirror within 8, mirror within 16), so each step adds the same two
// operands in either order and all 16 lanes hold identical bits; the four
// row sums are then read as scalars and added in a fixed order. DPP moves are
// VALU operations, several times quicker than LDS-routed shuffles.
__device__ __forceinline__ float wave_sum(float v) {
    v = v + dpp_mov<0xb1>(v);   // quad_perm [1,0,3,2]
    v = v + dpp_mov<0x4e>(v);   // quad_perm [2,3,0,1]
    v = v + dpp_mov<0x141>(v);  // row_half_mirror
    v = v + dpp_mov<0x140>(v);  // row_mirror
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// ─────────────────────────────── host side ───────────────────────────────
// Compute units of the current device (cached per device); 0 if unknown.
__attribute__((visibility("hidden"))) int device_cu_count();

inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }
inline bool is_float_dtype(int dt) { return dt == SPH_F32 || dt == SPH_F16 || dt == SPH_BF16; }
inline size_t dtype_size(int dt) { return dt == SPH_F32 ? 4 : 2; }

// Enqueue one launch of `kernel` and return that launch's own status.
// hipLaunchKernel reports the launch's error directly; reading hipGetLastError
// after a triple-chevron launch would also return (and clear) an error that an
// earlier, unrelated HIP call left on this thread. Arguments are converted to
// the kernel's parameter types, as a call would convert them.
template <typename... KArgs, typename... Args>
inline int launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t stream, Args&&... args) {
    static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count");
    std::tuple<KArgs...> vals(static_cast<KArgs>(std::forward<Args>(args))...);
    void* ptrs[sizeof...(KArgs)];
    std::apply([&ptrs](auto&... v) {
        int i = 0;
        ((ptrs[i++] = static_cast<void*>(&v)), ...);
    }, vals);
    return hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, ptrs, 0, stream) == hipSuccess
               ? SPH_OK
               : SPH_EHIP;
}

// Dispatch a functor templated on the storage type of a float dtype code.
template <typename F>
inline int with_float_type(int dt, F&& f) {
    switch (dt) {
    case SPH_F32: return f(float{});
    case SPH_F16: return f(f16{});
    case SPH_BF16: return f(bf16{});
    default: return SPH_EINVAL;
    }
}

}  // namespace sph
