// rmsnorm.hip — RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// Reference math (crates/sapient-backends/cpu/src/kernels/layernorm.rs:93-103):
//   ms = (Σ x_i²) / dim;  inv = 1 / sqrt(ms + eps);  y_i = (x_i · inv) · w_i
// The fused variant replaces `add` (llama.rs:508) followed by `rms_norm`
// (llama.rs:515): r = x + residual is written back to `residual` and y is the
// RMSNorm of the f32 sum.
//
// Design (HBM-bound, ≈0.2 flop/byte):
//  - A row is split across W wave64s (W = 1, 2, 4, 8 or 16, chosen so every
//    lane holds ~16 values); wave w owns the w-th contiguous 1/W of the row
//    (VPT runs of 64 16-byte vectors; contiguous chunks measured ~5 % faster
//    than interleaving the waves) and keeps its slice of r in registers, so
//    every input byte crosses HBM once and the row is never re-read. The
//    register footprint stays at ~64 VGPRs: the full 8 waves per SIMD.
//  - Each wave sums its r² with a butterfly of cross-lane shuffles; the W
//    partial sums meet in LDS and every wave adds them in the same fixed order.
//  - All row traffic is 16 bytes per lane (1 KiB contiguous per wave
//    instruction) and non-temporal: x, residual and y are touched once, and
//    streaming them past the caches measured ~+20 % achieved bandwidth on
//    MI355X. The weight row uses ordinary loads (it is re-read by every row).
//  - The residual store is issued before the reduction, overlapping it.
//  - Rows wider than 16 waves x 16 values, or whose pointers / width do not
//    allow 16-byte access, take a block-per-row two-pass kernel.
//
// Parity: x·x, the division by dim, sqrt and 1/· are IEEE-rounded f32 exactly
// as in the reference; the products y = (r·inv)·w round in the same order (the
// file is compiled with -ffp-contract=off). Only the order of the Σ differs
// (per-lane serial, then a tree), which moves ms by a few f32 ulps.
#include "sph_common.h"

namespace sph {
namespace {

constexpr int kWave = 64;

// W waves per row, VPT 16-byte vectors per lane, RPB rows per block.
template <typename TX, typename TW, typename TO, bool FUSED, int W, int VPT>
__global__ __launch_bounds__(W >= 4 ? 64 * W : 256) void rms_rows_vec(const TX* __restrict__ x, TX* __restrict__ residual,
                                                                   const TW* __restrict__ w, TO* __restrict__ out,
                                                                   int64_t rows, int dim, float eps) {
    constexpr int E = vec16<TX>::n;  // elements per 16-byte access of x
    constexpr int WPB = W >= 4 ? W : 4;
    constexpr int RPB = WPB / W;
    __shared__ float partial[WPB];
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave;
    const int sub = wv % W;  // this wave's share of the row
    const int64_t row = (int64_t)blockIdx.x * RPB + wv / W;
    const bool live = row < rows;
    const int nvec = dim / E;
    const size_t base = (size_t)row * (size_t)dim;

    float r[VPT][E];
    float ss = 0.0f;
    if (live) {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int v = (sub * VPT + j) * kWave + lane;
            if (v < nvec) {
                load_f32<TX, E, true>(x + base + (size_t)v * E, r[j]);
                if constexpr (FUSED) {
                    float b[E];
                    load_f32<TX, E, true>(residual + base + (size_t)v * E, b);
#pragma unroll
                    for (int e = 0; e < E; ++e) r[j][e] = r[j][e] + b[e];
                    store_f32<TX, E, true>(residual + base + (size_t)v * E, r[j]);
                }
#pragma unroll
                for (int e = 0; e < E; ++e) ss = ss + r[j][e] * r[j][e];
            }
        }
    }
    ss = wave_sum(ss);
    if constexpr (W > 1) {
        if (lane == 0) partial[wv] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int k = 0; k < W; ++k) tot = tot + partial[(wv / W) * W + k];
        ss = tot;
    }
    if (!live) return;
    const float ms = ss / (float)dim;
    const float inv = 1.0f / sqrtf(ms + eps);

#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int v = (sub * VPT + j) * kWave + lane;
        if (v < nvec) {
            float wv_[E];
            if (w != nullptr) {
                load_f32<TW, E>(w + (size_t)v * E, wv_);
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) wv_[e] = 1.0f;
            }
            float y[E];
#pragma unroll
            for (int e = 0; e < E; ++e) y[e] = (r[j][e] * inv) * wv_[e];
            store_f32<TO, E, true>(out + base + (size_t)v * E, y);
        }
    }
}

// Any width and alignment: one 256-thread block per row, two passes. Pass 2
// recomputes r from the inputs (it re-reads them from cache) so the half
// variants normalise the unrounded f32 sum; each thread owns the same
// elements in both passes, so the in-place residual update cannot race.
template <typename TX, typename TW, typename TO, bool FUSED>
__global__ __launch_bounds__(256) void rms_rows_generic(const TX* __restrict__ x, TX* residual,
                                                       const TW* __restrict__ w, TO* __restrict__ out,
                                                       int64_t rows, int64_t dim, float eps) {
    __shared__ float partial[256 / kWave];
    const int64_t row = blockIdx.x;
    const size_t base = (size_t)row * (size_t)dim;
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) {
        float r = widen(x[base + i]);
        if constexpr (FUSED) r = r + widen(residual[base + i]);
        ss = ss + r * r;
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & (kWave - 1)) == 0) partial[threadIdx.x / kWave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < 256 / kWave; ++i) tot = tot + partial[i];
    const float ms = tot / (float)dim;
    const float inv = 1.0f / sqrtf(ms + eps);
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) {
        float r = widen(x[base + i]);
        if constexpr (FUSED) {
            r = r + widen(residual[base + i]);
            residual[base + i] = narrow<TX>(r);
        }
        const float wv = w != nullptr ? widen(w[i]) : 1.0f;
        out[base + i] = narrow<TO>((r * inv) * wv);
    }
}

template <typename TX, typename TW, typename TO, bool FUSED>
int launch_rms(const void* x, void* residual, const void* w, void* out, int64_t rows, int64_t dim,
               float eps, hipStream_t stream) {
    if (rows == 0 || dim == 0) return SPH_OK;
    constexpr int E = vec16<TX>::n;
    // Vector path: ~16 values per lane, W waves per row (W <= 16).
    constexpr int VPT = 16 / E;
    const int64_t nvec = dim / E;
    int W = 1;
    while (W < 16 && nvec > (int64_t)kWave * VPT * W) W *= 2;
    const bool vec_ok = dim % E == 0 && aligned(x, 16) && aligned(out, 16) &&
                        (!FUSED || aligned(residual, 16)) && (w == nullptr || aligned(w, 16)) &&
                        nvec <= (int64_t)kWave * VPT * W && dim <= INT32_MAX;
    // A launch covers at most 2^22 rows, keeping grid x block below 2^32 work-items.
    constexpr int64_t kChunk = int64_t(1) << 22;
    for (int64_t r0 = 0; r0 < rows; r0 += kChunk) {
        const int64_t nr = rows - r0 < kChunk ? rows - r0 : kChunk;
        const size_t off = (size_t)r0 * (size_t)dim;
        const TX* xp = static_cast<const TX*>(x) + off;
        TX* rp = FUSED ? static_cast<TX*>(residual) + off : nullptr;
        const TW* wp = static_cast<const TW*>(w);
        TO* op = static_cast<TO*>(out) + off;
        if (vec_ok) {
            const int rpb = W >= 4 ? 1 : 4 / W;
            const dim3 grid((unsigned)((nr + rpb - 1) / rpb));
            const int threads = W >= 4 ? kWave * W : 256;
            const int d = (int)dim;
            switch (W) {
            case 1: rms_rows_vec<TX, TW, TO, FUSED, 1, VPT><<<grid, threads, 0, stream>>>(xp, rp, wp, op, nr, d, eps); break;
            case 2: rms_rows_vec<TX, TW, TO, FUSED, 2, VPT><<<grid, threads, 0, stream>>>(xp, rp, wp, op, nr, d, eps); break;
            case 4: rms_rows_vec<TX, TW, TO, FUSED, 4, VPT><<<grid, threads, 0, stream>>>(xp, rp, wp, op, nr, d, eps); break;
            case 8: rms_rows_vec<TX, TW, TO, FUSED, 8, VPT><<<grid, threads, 0, stream>>>(xp, rp, wp, op, nr, d, eps); break;
            default: rms_rows_vec<TX, TW, TO, FUSED, 16, VPT><<<grid, threads, 0, stream>>>(xp, rp, wp, op, nr, d, eps); break;
            }
        } else {
            rms_rows_generic<TX, TW, TO, FUSED><<<dim3((unsigned)nr), 256, 0, stream>>>(xp, rp, wp, op, nr, dim, eps);
        }
        const int st = launch_status();
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

// Resolve (x, weight, out) storage types: weight and out are each f32 or x's type.
template <bool FUSED>
int dispatch_rms(const void* x, void* residual, int x_dt, const void* w, int w_dt, void* out, int out_dt,
                 int64_t rows, int64_t dim, float eps, hipStream_t stream) {
    if (!is_float_dtype(x_dt)) return SPH_EINVAL;
    if (w != nullptr && w_dt != SPH_F32 && w_dt != x_dt) return SPH_EINVAL;
    if (out_dt != SPH_F32 && out_dt != x_dt) return SPH_EINVAL;
    const bool w32 = (w == nullptr) || w_dt == SPH_F32;
    const bool o32 = out_dt == SPH_F32;
    return with_float_type(x_dt, [&](auto tx) -> int {
        using TX = decltype(tx);
        if constexpr (sizeof(TX) == 4) {
            return launch_rms<float, float, float, FUSED>(x, residual, w, out, rows, dim, eps, stream);
        } else {
            if (w32 && o32) return launch_rms<TX, float, float, FUSED>(x, residual, w, out, rows, dim, eps, stream);
            if (w32 && !o32) return launch_rms<TX, float, TX, FUSED>(x, residual, w, out, rows, dim, eps, stream);
            if (!w32 && o32) return launch_rms<TX, TX, float, FUSED>(x, residual, w, out, rows, dim, eps, stream);
            return launch_rms<TX, TX, TX, FUSED>(x, residual, w, out, rows, dim, eps, stream);
        }
    });
}

}  // namespace
}  // namespace sph

extern "C" int sph_rms_norm(const void* x, int x_dtype, const void* weight, int w_dtype, void* out,
                            int out_dtype, int64_t rows, int64_t dim, float eps, void* stream) {
    if (rows < 0 || dim < 0) return SPH_EINVAL;
    if ((rows > 0 && dim > 0) && (x == nullptr || out == nullptr)) return SPH_EINVAL;
    return sph::dispatch_rms<false>(x, nullptr, x_dtype, weight, w_dtype, out, out_dtype, rows, dim, eps,
                                    static_cast<hipStream_t>(stream));
}

extern "C" int sph_add_rms_norm(const void* x, void* residual, int dtype, const void* weight, int w_dtype,
                                void* out, int out_dtype, int64_t rows, int64_t dim, float eps, void* stream) {
    if (rows < 0 || dim < 0) return SPH_EINVAL;
    if ((rows > 0 && dim > 0) && (x == nullptr || residual == nullptr || out == nullptr)) return SPH_EINVAL;
    if (out == x || out == residual) return SPH_EINVAL;
    return sph::dispatch_rms<true>(x, residual, dtype, weight, w_dtype, out, out_dtype, rows, dim, eps,
                                   static_cast<hipStream_t>(stream));
}
