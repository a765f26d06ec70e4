// rmsnorm.hip — RMSNorm, fused residual-add + RMSNorm and LayerNorm for gfx950.
//
// Reference math (crates/sapient-backends/cpu/src/kernels/layernorm.rs:93-103):
//   ms = (Σ x_i²) / dim;  inv = 1 / sqrt(ms + eps);  y_i = (x_i · inv) · w_i
// The fused variant replaces `add` (llama.rs:508) followed by `rms_norm`
// (llama.rs:515): r = x + residual is written back to `residual` (or, in the
// out-of-place form, to a separate `sum`) and y is the RMSNorm of the f32 sum. LayerNorm (layernorm.rs:17-69, last axis):
//   mean = Σx / n;  var = Σ(x − mean)² / n;  y = ((x − mean) · 1/sqrt(var + eps)) · w + b
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

// K_ADD_RMS writes the sum back into `residual`; K_ADD_RMS_TO writes it to `sum` and only reads
// `residual`.
enum Kind { K_RMS = 0, K_ADD_RMS = 1, K_LAYER = 2, K_ADD_RMS_TO = 3 };

constexpr bool adds(int kind) { return kind == K_ADD_RMS || kind == K_ADD_RMS_TO; }

// y for one element: RMSNorm (r·inv)·w; LayerNorm (d·inv)·w + b, where the
// caller passes the centred value d = r − mean for LayerNorm. An absent weight
// is passed as 1 and an absent bias as −0: x·1 and x + (−0) are x exactly
// (signed zeros included, where + (+0) would turn −0 into +0), so one
// branch-free expression gives each of the reference's four forms bit for bit.
template <int KIND>
__device__ __forceinline__ float norm_out(float r, float inv, float w, float b) {
    if constexpr (KIND == K_LAYER) return (r * inv) * w + b;
    else return (r * inv) * w;
}

// Sum of one value per wave of a row: the W partials meet in LDS and every
// wave adds them in the same order. `slot` lets two reductions share a barrier-safe buffer.
template <int W, int WPB>
__device__ __forceinline__ float row_sum(float v, float (*partial)[WPB], int slot, int lane, int wv) {
    v = wave_sum(v);
    if constexpr (W > 1) {
        if (lane == 0) partial[slot][wv] = v;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int k = 0; k < W; ++k) tot = tot + partial[slot][(wv / W) * W + k];
        v = tot;
    }
    return v;
}

// 16 bytes of T as f32 values.
template <typename T, int E>
__device__ __forceinline__ void unpack16(const u32x4& q, float (&v)[E]) {
    const uint32_t raw[4] = {q.x, q.y, q.z, q.w};
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(raw[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = widen(T{(uint16_t)(raw[i / 2] >> (16 * (i & 1)))});
    }
}

// W waves per row, VPT 16-byte vectors per lane, RPB rows per block.
//  LOOP = false: block b owns row b·RPB + wave/W; weight and bias are read at
//    the output stage (the lowest register footprint).
//  LOOP = true: block b walks rows b·RPB, + step, ... (step = gridDim.x · RPB)
//    with weight and bias held in registers across its rows and the next
//    row's raw vectors loaded before the current row is reduced. Used where a
//    grid of a few blocks per CU re-reads the weights less than one block per
//    row would (LayerNorm: weight and bias rows).
template <typename TX, typename TW, typename TO, int KIND, int W, int VPT, bool LOOP>
__global__ __launch_bounds__(W >= 4 ? 64 * W : 256) void rms_rows_vec(const TX* __restrict__ x, TX* __restrict__ residual,
                                                                   TX* __restrict__ sum, const TW* __restrict__ w,
                                                                   const TW* __restrict__ bias, TO* __restrict__ out,
                                                                   int64_t rows, int dim, float eps) {
    constexpr int E = vec16<TX>::n;  // elements per 16-byte access of x
    constexpr int WPB = W >= 4 ? W : 4;
    constexpr int RPB = WPB / W;
    // Two buffers, alternating by row: a wave still reading row i's partials
    // cannot be overtaken by row i + 2's writes (row i + 1's barrier lies between).
    __shared__ float partial[2][2][WPB];
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave;
    const int sub = wv % W;  // this wave's share of the row
    const int nvec = dim / E;
    const bool has_w = w != nullptr, has_b = bias != nullptr;

    auto load_wb = [&](int j, float (&wj)[E], float (&bj)[E]) {
        const int v = (sub * VPT + j) * kWave + lane;
        if (v < nvec && has_w) {
            load_f32<TW, E>(w + (size_t)v * E, wj);
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) wj[e] = 1.0f;
        }
        if (v < nvec && KIND == K_LAYER && has_b) {
            load_f32<TW, E>(bias + (size_t)v * E, bj);
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) bj[e] = -0.0f;
        }
    };
    auto fetch = [&](int64_t row, u32x4 (&vx)[VPT], u32x4 (&vres)[VPT]) {
        if (row >= rows) return;
        const size_t base = (size_t)row * (size_t)dim;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int v = (sub * VPT + j) * kWave + lane;
            if (v < nvec) {
                vx[j] = vload<true>(reinterpret_cast<const u32x4*>(x + base + (size_t)v * E));
                if constexpr (adds(KIND))
                    vres[j] = vload<true>(reinterpret_cast<const u32x4*>(residual + base + (size_t)v * E));
            }
        }
    };
    // One row from its raw vectors: sums, reductions, output. `wr`/`br` are
    // the held weights (LOOP) or unused (weights read at the output stage).
    auto row_body = [&](int64_t row, const u32x4 (&cx)[VPT], const u32x4 (&cres)[VPT], int par,
                        const float (*wr)[E], const float (*br)[E]) {
        const bool live = row < rows;
        const size_t base = (size_t)row * (size_t)dim;
        float r[VPT][E];
        float ss = 0.0f;
        if (live) {
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const int v = (sub * VPT + j) * kWave + lane;
                if (v < nvec) {
                    unpack16<TX, E>(cx[j], r[j]);
                    if constexpr (adds(KIND)) {
                        float b[E];
                        unpack16<TX, E>(cres[j], b);
#pragma unroll
                        for (int e = 0; e < E; ++e) r[j][e] = r[j][e] + b[e];
                        store_f32<TX, E, true>((KIND == K_ADD_RMS_TO ? sum : residual) + base + (size_t)v * E, r[j]);
                    }
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        if constexpr (KIND == K_LAYER) ss = ss + r[j][e];
                        else ss = ss + r[j][e] * r[j][e];
                    }
                }
            }
        }
        ss = row_sum<W, WPB>(ss, partial[par], 0, lane, wv);
        float inv;
        if constexpr (KIND == K_LAYER) {
            // The row is centred once, in registers: the variance and the
            // output both use d = r − mean (the same f32 difference each time).
            const float mean = ss / (float)dim;
            float vs = 0.0f;
            if (live) {
#pragma unroll
                for (int j = 0; j < VPT; ++j) {
                    const int v = (sub * VPT + j) * kWave + lane;
                    if (v < nvec) {
#pragma unroll
                        for (int e = 0; e < E; ++e) {
                            r[j][e] = r[j][e] - mean;
                            vs = vs + r[j][e] * r[j][e];
                        }
                    }
                }
            }
            vs = row_sum<W, WPB>(vs, partial[par], 1, lane, wv);
            inv = 1.0f / sqrtf(vs / (float)dim + eps);
        } else {
            inv = 1.0f / sqrtf(ss / (float)dim + eps);
        }
        if (!live) return;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int v = (sub * VPT + j) * kWave + lane;
            if (v < nvec) {
                float wj[E], bj[E];
                if constexpr (LOOP) {
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        wj[e] = wr[j][e];
                        bj[e] = br[j][e];
                    }
                } else {
                    load_wb(j, wj, bj);
                }
                float y[E];
#pragma unroll
                for (int e = 0; e < E; ++e) y[e] = norm_out<KIND>(r[j][e], inv, wj[e], bj[e]);
                store_f32<TO, E, true>(out + base + (size_t)v * E, y);
            }
        }
    };

    const int64_t first = (int64_t)blockIdx.x * RPB;
    if constexpr (!LOOP) {
        u32x4 cx[VPT], cres[VPT];
        fetch(first + wv / W, cx, cres);
        row_body(first + wv / W, cx, cres, 0, nullptr, nullptr);
    } else {
        float wr[VPT][E], br[VPT][E];
#pragma unroll
        for (int j = 0; j < VPT; ++j) load_wb(j, wr[j], br[j]);
        const int64_t step = (int64_t)gridDim.x * RPB;
        u32x4 nx[VPT], nres[VPT];
        fetch(first + wv / W, nx, nres);
        int par = 0;
        for (int64_t row0 = first; row0 < rows; row0 += step, par ^= 1) {  // trip count uniform over the block
            const int64_t row = row0 + wv / W;
            u32x4 cx[VPT], cres[VPT];
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                cx[j] = nx[j];
                cres[j] = nres[j];
            }
            fetch(row + step, nx, nres);
            row_body(row, cx, cres, par, wr, br);
        }
    }
}

// Any width and alignment: one 256-thread block per row, re-reading the row
// from cache for each pass. The last pass recomputes r from the inputs so the
// half variants normalise the unrounded f32 sum; each thread owns the same
// elements in every pass, so the in-place residual update cannot race.
template <typename TX, typename TW, typename TO, int KIND>
__global__ __launch_bounds__(256) void rms_rows_generic(const TX* __restrict__ x, TX* residual, TX* __restrict__ sum,
                                                       const TW* __restrict__ w, const TW* __restrict__ bias,
                                                       TO* __restrict__ out, int64_t rows, int64_t dim, float eps) {
    __shared__ float partial[2][256 / kWave];
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
    const int64_t row = blockIdx.x;
    if (row >= rows) return;  // the grid is one block per row; block-uniform, before any barrier
    const size_t base = (size_t)row * (size_t)dim;
    auto value = [&](int64_t i) {
        float r = widen(x[base + i]);
        if constexpr (adds(KIND)) r = r + widen(residual[base + i]);
        return r;
    };
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) {
        const float r = value(i);
        if constexpr (KIND == K_LAYER) ss = ss + r;
        else ss = ss + r * r;
    }
    ss = row_sum<4, 4>(ss, partial, 0, lane, wv);
    float mean = 0.0f, inv;
    if constexpr (KIND == K_LAYER) {
        mean = ss / (float)dim;
        float vs = 0.0f;
        for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) {
            const float d = value(i) - mean;
            vs = vs + d * d;
        }
        vs = row_sum<4, 4>(vs, partial, 1, lane, wv);
        inv = 1.0f / sqrtf(vs / (float)dim + eps);
    } else {
        inv = 1.0f / sqrtf(ss / (float)dim + eps);
    }
    const bool has_w = w != nullptr, has_b = bias != nullptr;
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) {
        const float r = value(i);
        if constexpr (KIND == K_ADD_RMS) residual[base + i] = narrow<TX>(r);
        if constexpr (KIND == K_ADD_RMS_TO) sum[base + i] = narrow<TX>(r);
        const float wv_ = has_w ? widen(w[i]) : 1.0f;
        const float bv = (KIND == K_LAYER && has_b) ? widen(bias[i]) : -0.0f;
        out[base + i] = narrow<TO>(norm_out<KIND>(KIND == K_LAYER ? r - mean : r, inv, wv_, bv));
    }
}

template <typename TX, typename TW, typename TO, int KIND, int VPT, bool LOOP>
int launch_vec(int W, dim3 grid, int threads, const TX* xp, TX* rp, TX* sp, const TW* wp, const TW* bp, TO* op,
               int64_t nr, int d, float eps, hipStream_t stream) {
    switch (W) {
    case 1: return launch(rms_rows_vec<TX, TW, TO, KIND, 1, VPT, LOOP>, grid, threads, stream, xp, rp, sp, wp, bp, op, nr, d, eps);
    case 2: return launch(rms_rows_vec<TX, TW, TO, KIND, 2, VPT, LOOP>, grid, threads, stream, xp, rp, sp, wp, bp, op, nr, d, eps);
    case 4: return launch(rms_rows_vec<TX, TW, TO, KIND, 4, VPT, LOOP>, grid, threads, stream, xp, rp, sp, wp, bp, op, nr, d, eps);
    case 8: return launch(rms_rows_vec<TX, TW, TO, KIND, 8, VPT, LOOP>, grid, threads, stream, xp, rp, sp, wp, bp, op, nr, d, eps);
    default: return launch(rms_rows_vec<TX, TW, TO, KIND, 16, VPT, LOOP>, grid, threads, stream, xp, rp, sp, wp, bp, op, nr, d, eps);
    }
}

// launch_shape's result when the shape does not cover the row (nothing launched).
constexpr int kNoShape = 1;

// One launch of the vector kernel with VPT 16-byte vectors per lane: W waves
// per row (the fewest that cover it), LOOP blocks capped at `waves_per_cu`
// resident waves per CU (at least one block). Returns the launch's status, or
// kNoShape, launching nothing, when a row is wider than 16 waves cover.
template <typename TX, typename TW, typename TO, int KIND, int VPT, bool LOOP>
int launch_shape(const TX* xp, TX* rp, TX* sp, const TW* wp, const TW* bp, TO* op, int64_t nr, int dim, float eps,
                  int waves_per_cu, hipStream_t stream) {
    constexpr int E = vec16<TX>::n;
    const int64_t nvec = dim / E;
    int W = 1;
    while (W < 16 && nvec > (int64_t)kWave * VPT * W) W *= 2;
    if (nvec > (int64_t)kWave * VPT * W) return kNoShape;
    const int rpb = W >= 4 ? 1 : 4 / W;
    const int threads = W >= 4 ? kWave * W : 256;
    int64_t nb = (nr + rpb - 1) / rpb;
    if (LOOP) {
        const int cus = device_cu_count();
        const int per_cu = waves_per_cu / (threads / kWave);
        if (cus > 0) {
            const int64_t cap = (int64_t)cus * (per_cu > 1 ? per_cu : 1);
            if (nb > cap) nb = cap;
        }
    }
    return launch_vec<TX, TW, TO, KIND, VPT, LOOP>(W, dim3((unsigned)nb), threads, xp, rp, sp, wp, bp, op, nr, dim, eps,
                                                   stream);
}

// Launch shapes, measured at 16384 x 4096 on MI355X (round-robin medians on
// two machines; one-block-per-row shapes listed as VPT):
//  - fused add + RMSNorm: row-looping blocks, one vector per lane, 16 (f32)
//    or 8 (half) resident waves per CU: f32 171.8 µs (one block per row,
//    VPT 2: 175.0), f16 85.4 µs (VPT 1: 87.6), bf16 85.8 µs (84.9);
//  - plain RMSNorm, half: row-looping, four vectors per lane, 8 resident
//    waves per CU: f16 44.6 µs, bf16 47.0 (one block per row: 47.0, 48.7;
//    two vectors per lane looping: 44.8, 54.5);
//  - plain RMSNorm, f32: one block per row, two vectors per lane (85.0 µs;
//    looping: 86.8);
//  - LayerNorm: row-looping with weight and bias held in registers, 8 resident
//    waves per CU, two (f32) or four (half) vectors per lane: f32 85.9 µs,
//    f16 47.4 µs (16 waves per CU with two vectors: 88.8, 48.9; one block per
//    row: 92.0, 55.6).
// A row too wide for the looping shape takes the one-block-per-row kernel
// (twice the values per lane past 16 waves); unaligned rows, or rows wider
// than that, the generic kernel.
constexpr int64_t kFewValues = int64_t(1) << 21;

template <typename TX, typename TW, typename TO, int KIND>
int launch_rms(const void* x, void* residual, void* sum, const void* w, const void* bias, void* out, int64_t rows,
               int64_t dim, float eps, hipStream_t stream) {
    if (rows == 0 || dim == 0) return SPH_OK;
    constexpr int E = vec16<TX>::n;
    constexpr bool FUSED = adds(KIND);
    constexpr bool HALF = sizeof(TX) == 2;
    // One-block-per-row (or LayerNorm's looping) shape: values per lane.
    constexpr int VPT = (HALF && !FUSED) ? 2 : 8 / E;
    constexpr bool kLoop = KIND == K_LAYER;
    // The row-looping shape tried first (VPT_L values per lane, 0: none) and its
    // resident waves per CU.
    constexpr int VPT_L = FUSED ? 1 : (HALF ? 4 : (KIND == K_LAYER ? 2 : 0));
    constexpr int kLoopWaves = FUSED && !HALF ? 16 : 8;
    const int64_t nvec = dim / E;
    const bool vec_ok = dim % E == 0 && aligned(x, 16) && aligned(out, 16) &&
                        (!FUSED || aligned(residual, 16)) && (KIND != K_ADD_RMS_TO || aligned(sum, 16)) &&
                        (w == nullptr || aligned(w, 16)) &&
                        (bias == nullptr || aligned(bias, 16)) && nvec <= (int64_t)kWave * 2 * VPT * 16 &&
                        dim <= INT32_MAX;
    // A launch covers at most 2^22 rows, keeping grid x block below 2^32 work-items.
    constexpr int64_t kChunk = int64_t(1) << 22;
    for (int64_t r0 = 0; r0 < rows; r0 += kChunk) {
        const int64_t nr = rows - r0 < kChunk ? rows - r0 : kChunk;
        const size_t off = (size_t)r0 * (size_t)dim;
        const TX* xp = static_cast<const TX*>(x) + off;
        TX* rp = FUSED ? static_cast<TX*>(residual) + off : nullptr;
        TX* sp = KIND == K_ADD_RMS_TO ? static_cast<TX*>(sum) + off : nullptr;
        const TW* wp = static_cast<const TW*>(w);
        const TW* bp = static_cast<const TW*>(bias);
        TO* op = static_cast<TO*>(out) + off;
        int st = kNoShape;
        if (vec_ok) {
            // Launches of up to 2^21 values (a decode step, a prefill chunk at small widths): one
            // vector per lane and twice the waves per row, so each wave's chain is one load
            // before its reduction. Back-to-back per launch on MI355X, against the shapes below:
            // 1 x 896 f32 1.87 -> 1.65 µs, f16 2.10 -> 1.65; 512 x 896 f32 2.73 -> 2.36-2.46,
            // f16 2.89 -> 2.34; 512 x 4096 f16 3.6 -> 2.9, f32 3.83 -> 3.63; at 2048 x 4096 it
            // lost (f16 6.7 -> 7.9, f32 12.9 -> 13.7), hence the bound.
            if constexpr ((KIND == K_RMS || KIND == K_LAYER) && VPT > 1)
                if (nr * dim <= kFewValues)
                    st = launch_shape<TX, TW, TO, KIND, 1, false>(xp, rp, sp, wp, bp, op, nr, (int)dim, eps, 16, stream);
            if constexpr (VPT_L > 0)
                if (st == kNoShape)
                    st = launch_shape<TX, TW, TO, KIND, VPT_L, true>(xp, rp, sp, wp, bp, op, nr, (int)dim, eps,
                                                                     kLoopWaves, stream);
            if (st == kNoShape)
                st = launch_shape<TX, TW, TO, KIND, VPT, kLoop>(xp, rp, sp, wp, bp, op, nr, (int)dim, eps, 16, stream);
            if (st == kNoShape)  // wider than 16 waves at VPT: twice the values per lane, one block per row
                st = launch_shape<TX, TW, TO, KIND, 2 * VPT, false>(xp, rp, sp, wp, bp, op, nr, (int)dim, eps, 16, stream);
            if (st == kNoShape) return SPH_EINVAL;  // unreachable: vec_ok bounds the width
        } else {
            st = launch(rms_rows_generic<TX, TW, TO, KIND>, dim3((unsigned)nr), 256, stream, xp, rp, sp, wp, bp, op,
                        nr, dim, eps);
        }
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

// Resolve (x, weight/bias, out) storage types: weight/bias and out are each f32 or x's type.
template <int KIND>
int dispatch_rms(const void* x, void* residual, void* sum, int x_dt, const void* w, const void* b, int w_dt, void* out,
                 int out_dt, int64_t rows, int64_t dim, float eps, hipStream_t stream) {
    if (!is_float_dtype(x_dt)) return SPH_EINVAL;
    if ((w != nullptr || b != nullptr) && w_dt != SPH_F32 && w_dt != x_dt) return SPH_EINVAL;
    if (out_dt != SPH_F32 && out_dt != x_dt) return SPH_EINVAL;
    const bool w32 = (w == nullptr && b == nullptr) || w_dt == SPH_F32;
    const bool o32 = out_dt == SPH_F32;
    return with_float_type(x_dt, [&](auto tx) -> int {
        using TX = decltype(tx);
        if constexpr (sizeof(TX) == 4) {
            return launch_rms<float, float, float, KIND>(x, residual, sum, w, b, out, rows, dim, eps, stream);
        } else {
            if (w32 && o32) return launch_rms<TX, float, float, KIND>(x, residual, sum, w, b, out, rows, dim, eps, stream);
            if (w32 && !o32) return launch_rms<TX, float, TX, KIND>(x, residual, sum, w, b, out, rows, dim, eps, stream);
            if (!w32 && o32) return launch_rms<TX, TX, float, KIND>(x, residual, sum, w, b, out, rows, dim, eps, stream);
            return launch_rms<TX, TX, TX, KIND>(x, residual, sum, w, b, out, rows, dim, eps, stream);
        }
    });
}

}  // namespace
}  // namespace sph

extern "C" int sph_rms_norm(const void* x, int x_dtype, const void* weight, int w_dtype, void* out,
                            int out_dtype, int64_t rows, int64_t dim, float eps, void* stream) {
    if (rows < 0 || dim < 0) return SPH_EINVAL;
    if ((rows > 0 && dim > 0) && (x == nullptr || out == nullptr)) return SPH_EINVAL;
    return sph::dispatch_rms<sph::K_RMS>(x, nullptr, nullptr, x_dtype, weight, nullptr, w_dtype, out, out_dtype, rows, dim, eps,
                                         static_cast<hipStream_t>(stream));
}

extern "C" int sph_add_rms_norm(const void* x, void* residual, int dtype, const void* weight, int w_dtype,
                                void* out, int out_dtype, int64_t rows, int64_t dim, float eps, void* stream) {
    if (rows < 0 || dim < 0) return SPH_EINVAL;
    if ((rows > 0 && dim > 0) && (x == nullptr || residual == nullptr || out == nullptr)) return SPH_EINVAL;
    if (out == x || out == residual) return SPH_EINVAL;
    return sph::dispatch_rms<sph::K_ADD_RMS>(x, residual, nullptr, dtype, weight, nullptr, w_dtype, out, out_dtype, rows,
                                             dim, eps, static_cast<hipStream_t>(stream));
}

extern "C" int sph_add_rms_norm_to(const void* x, const void* residual, void* sum, int dtype, const void* weight,
                                   int w_dtype, void* out, int out_dtype, int64_t rows, int64_t dim, float eps,
                                   void* stream) {
    if (sum == residual) return sph_add_rms_norm(x, sum, dtype, weight, w_dtype, out, out_dtype, rows, dim, eps, stream);
    if (rows < 0 || dim < 0) return SPH_EINVAL;
    if ((rows > 0 && dim > 0) && (x == nullptr || residual == nullptr || sum == nullptr || out == nullptr))
        return SPH_EINVAL;
    if (out == x || out == residual || out == sum || sum == x) return SPH_EINVAL;
    return sph::dispatch_rms<sph::K_ADD_RMS_TO>(x, const_cast<void*>(residual), sum, dtype, weight, nullptr, w_dtype,
                                                out, out_dtype, rows, dim, eps, static_cast<hipStream_t>(stream));
}

extern "C" int sph_layer_norm(const void* x, int x_dtype, const void* weight, const void* bias, int wb_dtype,
                              void* out, int out_dtype, int64_t rows, int64_t dim, float eps, void* stream) {
    if (rows < 0 || dim < 0) return SPH_EINVAL;
    if ((rows > 0 && dim > 0) && (x == nullptr || out == nullptr)) return SPH_EINVAL;
    return sph::dispatch_rms<sph::K_LAYER>(x, nullptr, nullptr, x_dtype, weight, bias, wb_dtype, out, out_dtype, rows, dim,
                                           eps, static_cast<hipStream_t>(stream));
}
