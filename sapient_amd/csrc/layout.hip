// layout.hip — the device-resident decode helpers: head transposes and the
// KV-cache append, for gfx950.
//
// Reference (crates/sapient-backends/wgpu/src/resident.rs):
//   transpose_heads  [outer, inner, hd] → [inner, outer, hd]          (:420-458)
//   kv_append        src [n_kv, seq, hd] → cache[:, pos:pos+seq, :]
//                    of [n_kv, max_seq, hd], converted to the cache type (:645-711)
//
// Both are moves of hd-element rows between two row orders, so one kernel
// serves both: each thread moves 16 bytes of the narrower side (f32: 4
// elements, halves: 8; an f32 → half move reads two 16-byte words and writes
// one; 16 bytes of the wider side when hd is not a multiple of 8),
// non-temporal, with a per-row index map. The transpose walks 8 × 8 tiles of
// (outer, inner) rows, so a block's reads cover 8 runs of 8 consecutive
// source rows and its writes 8 runs of 8 consecutive output rows (measured at
// [8192, 32, 128] f32: 72 µs walking output rows with two 16-byte accesses per
// thread, 47.5 µs with one, 45.3 µs with tiles). The append walks source rows
// (reads contiguous, writes contiguous within each head's run of seq rows).
// Same-type moves copy raw bits (NaN payloads included); f32 → f16 / bf16
// rounds to nearest-even, the conversion the reference's host mirror applies
// (half::f16::from_f32). HBM-bound: read + write once per element.
#include <type_traits>

#include "sph_common.h"

namespace sph {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kTile = 8;  // transpose tiles: 8 outer x 8 inner rows

enum Map { M_TRANSPOSE = 0, M_KV = 1 };

// Row index map. TRANSPOSE: a = outer, b = inner, row = a tile-ordered row
// index (see tile_row). KV: walk source rows r = h·seq + s, destination row
// h·max_seq + pos + s (a = seq, b = max_seq, c = pos).
struct RowMap {
    uint32_t a, b;
    uint64_t c;
};

// Rows of one call number fewer than 2^32 (checked on the host), so the
// splits are 32-bit divisions. Returns false for the padding rows of edge tiles.
template <int MAP>
__device__ __forceinline__ bool map_row(uint32_t row, const RowMap& m, uint64_t& srow, uint64_t& drow) {
    if constexpr (MAP == M_TRANSPOSE) {
        // row = tile · 64 + w; tiles in output order (inner-tile major), and
        // inside a tile w = wi · 8 + wo, so consecutive rows are consecutive outputs.
        const uint32_t tiles_o = (m.a + kTile - 1) / kTile;
        const uint32_t tile = row / (kTile * kTile), w = row % (kTile * kTile);
        const uint32_t ti = tile / tiles_o, to = tile - ti * tiles_o;
        const uint32_t o = to * kTile + w % kTile, i = ti * kTile + w / kTile;
        if (o >= m.a || i >= m.b) return false;
        srow = (uint64_t)o * m.b + i;
        drow = (uint64_t)i * m.a + o;
    } else {
        const uint32_t hi = row / m.a, lo = row - hi * m.a;
        srow = row;
        drow = (uint64_t)hi * m.b + m.c + lo;
    }
    return true;
}

// Elements per thread of the vector path: 16 bytes of the narrower side (an
// f32 <-> half move reads or writes two 16-byte words, so both sides stay
// 16 bytes wide), or, when hd is not a multiple of that, 16 bytes of the wider side.
template <typename TS, typename TD>
struct MoveWidth {
    static constexpr int wide = 16 / (int)(sizeof(TS) < sizeof(TD) ? sizeof(TS) : sizeof(TD));
    static constexpr int narrow = 16 / (int)(sizeof(TS) > sizeof(TD) ? sizeof(TS) : sizeof(TD));
};

template <typename TS, typename TD, int E>
__device__ __forceinline__ void move_chunk(const TS* s, TD* d) {
    if constexpr (std::is_same<TS, TD>::value) {
        vstore<true>(reinterpret_cast<u32x4*>(d), vload<true>(reinterpret_cast<const u32x4*>(s)));
    } else {
        float v[E];
        load_f32<TS, E, true>(s, v);
        store_f32<TD, E, true>(d, v);
    }
}

// Vector path: hd a multiple of the chunk width E, both bases 16-byte aligned;
// rows [row0, row0 + items / cpr) of this launch, cpr chunks per row.
template <typename TS, typename TD, int MAP, int E>
__global__ __launch_bounds__(kThreads) void move_rows_vec(const TS* __restrict__ src, TD* __restrict__ dst,
                                                          uint32_t items, uint32_t cpr, uint32_t row0, RowMap m) {
    const uint32_t k = blockIdx.x * kThreads + threadIdx.x;
    if (k >= items) return;
    const uint32_t r = k / cpr;
    const uint32_t c = (k - r * cpr) * E;
    uint64_t srow, drow;
    if (!map_row<MAP>(row0 + r, m, srow, drow)) return;
    const uint64_t hd = (uint64_t)cpr * E;
    move_chunk<TS, TD, E>(src + srow * hd + c, dst + drow * hd + c);
}

// Any hd / alignment: one element per thread.
template <typename TS, typename TD, int MAP>
__global__ __launch_bounds__(kThreads) void move_rows_scalar(const TS* __restrict__ src, TD* __restrict__ dst,
                                                             uint32_t items, uint32_t hd, uint32_t row0, RowMap m) {
    const uint32_t k = blockIdx.x * kThreads + threadIdx.x;
    if (k >= items) return;
    const uint32_t r = k / hd;
    const uint32_t c = k - r * hd;
    uint64_t srow, drow;
    if (!map_row<MAP>(row0 + r, m, srow, drow)) return;
    if constexpr (std::is_same<TS, TD>::value) dst[drow * hd + c] = src[srow * hd + c];
    else dst[drow * hd + c] = narrow<TD>(widen(src[srow * hd + c]));
}

// `rows` = rows of the walk (the transpose's includes edge-tile padding).
template <typename TS, typename TD, int MAP>
int launch_move(const void* src, void* dst, uint64_t rows, uint64_t hd, RowMap m, hipStream_t stream) {
    if (rows == 0 || hd == 0) return SPH_OK;
    if (hd > (1u << 24) || rows > UINT32_MAX) return SPH_EINVAL;
    constexpr int EW = MoveWidth<TS, TD>::wide, EN = MoveWidth<TS, TD>::narrow;
    const TS* s = static_cast<const TS*>(src);
    TD* d = static_cast<TD*>(dst);
    const bool al = aligned(src, 16) && aligned(dst, 16);
    const int E = !al ? 0 : hd % EW == 0 ? EW : hd % EN == 0 ? EN : 0;  // 0: scalar path
    const uint64_t per_row = E ? hd / E : hd;  // work items per row
    // Each launch covers whole rows (whole tiles for the transpose) and fewer than 2^31 work items.
    uint64_t rows_per_launch = ((uint64_t)1 << 31) / per_row;
    if (MAP == M_TRANSPOSE) rows_per_launch -= rows_per_launch % (kTile * kTile);
    for (uint64_t r0 = 0; r0 < rows; r0 += rows_per_launch) {
        const uint64_t nr = rows - r0 < rows_per_launch ? rows - r0 : rows_per_launch;
        const uint32_t items = (uint32_t)(nr * per_row);
        const dim3 grid((items + kThreads - 1) / kThreads);
        const int st = E == EW ? launch(move_rows_vec<TS, TD, MAP, EW>, grid, kThreads, stream, s, d, items,
                                        (uint32_t)per_row, (uint32_t)r0, m)
                     : E == EN ? launch(move_rows_vec<TS, TD, MAP, EN>, grid, kThreads, stream, s, d, items,
                                        (uint32_t)per_row, (uint32_t)r0, m)
                               : launch(move_rows_scalar<TS, TD, MAP>, grid, kThreads, stream, s, d, items,
                                        (uint32_t)hd, (uint32_t)r0, m);
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

// Q8_0 cache: one thread per 32-element block of a (head, token) row, the
// quantizer of the reference's quantized KV cache
// (crates/sapient-models/src/forward/common.rs:336-348, the same steps as
// quant.rs:223-235): amax over the block (NaN skipped, as f32::max folds),
// scale = amax / 127 in f32, d = f16(scale), q = clamp(round(v · 1/scale),
// ±127) with round half away from zero and NaN → 0 (the `as i8` cast), and 0
// throughout for an all-zero block. Row layout: head_dim / 32 blocks of
// 34 bytes (f16 d, 32 × i8), rows of a head at positions 0 .. max_seq - 1.
template <typename TS>
__global__ __launch_bounds__(kThreads) void kv_append_q8_0(const TS* __restrict__ src, uint8_t* __restrict__ cache,
                                                           uint64_t blocks, uint32_t bpr, uint32_t seq,
                                                           uint32_t max_seq, uint64_t pos) {
    const uint64_t k = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (k >= blocks) return;
    const uint64_t row = k / bpr;                // source row h · seq + s
    const uint32_t blk = (uint32_t)(k - row * bpr);
    const uint64_t h = row / seq, s = row - h * seq;
    float v[32];
    load_f32<TS, 32>(src + row * (uint64_t)bpr * 32 + (uint64_t)blk * 32, v);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    const float scale = amax / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    uint8_t* out = cache + ((h * max_seq + pos + s) * (uint64_t)bpr + blk) * 34;  // 2-byte aligned
    uint16_t* o16 = reinterpret_cast<uint16_t*>(out);
    o16[0] = narrow<f16>(scale).bits;
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
        int8_t q[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float r = roundf(v[i + j] * inv);  // half away from zero
            q[j] = r != r ? (int8_t)0 : (int8_t)fminf(fmaxf(r, -127.0f), 127.0f);
        }
        o16[1 + i / 2] = (uint16_t)((uint8_t)q[0] | ((uint16_t)(uint8_t)q[1] << 8));
    }
}

// Sliding-window shift of a KV cache (the trait path's update_kv_cache,
// crates/sapient-models/src/forward/common.rs:392-405 and :475-485): in every
// head, rows [shift, cur_len) move to [0, keep), keep = cur_len - shift, in
// place; the `shift` rows after them are then overwritten by the append. With
// X = rows [0, shift) and Y = rows [shift, cur_len), reversing Y and then the
// whole of [0, cur_len) turns X Y into Y rev(X): Y lands in [0, keep) and
// rev(X) in the rows the append overwrites. A reversal is a set of disjoint
// row swaps (row lo + j with row hi - 1 - j), so every thread swaps its units
// on its own — no ordering between blocks, no scratch memory — and the kernel
// boundary orders the two passes. Each pass reads and writes every row once
// (twice the bytes of a direct move) in whole rows, coalesced, over the whole
// GPU; a direct in-place move must keep each column of a head in one block,
// since a row is read by the row `shift` below it (16 bytes per row access,
// 128 blocks): a one-token update of a full 8 x 8192 x 128 f16 cache took
// 31.7 us that way and 16.0 us with the two passes, the append included.
template <typename UT>
__global__ __launch_bounds__(kThreads) void kv_reverse_rows(UT* cache, uint32_t units_per_row, uint64_t max_seq,
                                                            uint64_t lo, uint64_t hi, uint32_t items) {
    // items = (hi - lo) / 2 pairs x units_per_row, per head (blockIdx.y).
    const uint32_t i = blockIdx.x * (uint32_t)kThreads + threadIdx.x;
    if (i >= items) return;
    const uint32_t j = i / units_per_row, u = i - j * units_per_row;
    UT* base = cache + (uint64_t)blockIdx.y * max_seq * units_per_row + u;
    UT* a = base + (lo + j) * units_per_row;
    UT* b = base + (hi - 1 - j) * units_per_row;
    const UT va = *a, vb = *b;
    *a = vb;
    *b = va;
}

template <typename UT>
int launch_reverse(void* cache, uint64_t n_heads, uint64_t row_bytes, uint64_t max_seq, uint64_t lo, uint64_t hi,
                   hipStream_t stream) {
    const uint64_t upr = row_bytes / sizeof(UT);
    const uint64_t items = (hi - lo) / 2 * upr;
    if (items == 0) return SPH_OK;
    if (items > UINT32_MAX - kThreads || upr > UINT32_MAX) return SPH_EINVAL;
    constexpr uint64_t kMaxY = 65535;  // heads per launch (grid y)
    for (uint64_t h0 = 0; h0 < n_heads; h0 += kMaxY) {
        const uint64_t nh = n_heads - h0 < kMaxY ? n_heads - h0 : kMaxY;
        const dim3 grid((unsigned)((items + kThreads - 1) / kThreads), (unsigned)nh);
        const int st = launch(kv_reverse_rows<UT>, grid, kThreads, stream,
                              static_cast<UT*>(cache) + h0 * max_seq * upr, (uint32_t)upr, max_seq, lo, hi,
                              (uint32_t)items);
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

// The two passes, with the widest unit the row width and the cache's alignment allow.
// The second pass covers more rows than the first, so checking its item count
// before either launch means a rejected shift leaves the cache untouched.
template <typename UT>
int shift_window(void* cache, uint64_t n_heads, uint64_t row_bytes, uint64_t max_seq, uint64_t shift,
                 uint64_t cur_len, hipStream_t stream) {
    const uint64_t upr = row_bytes / sizeof(UT);
    if (upr > UINT32_MAX || cur_len / 2 * upr > UINT32_MAX - kThreads) return SPH_EINVAL;
    const int st = launch_reverse<UT>(cache, n_heads, row_bytes, max_seq, shift, cur_len, stream);
    if (st != SPH_OK) return st;
    return launch_reverse<UT>(cache, n_heads, row_bytes, max_seq, 0, cur_len, stream);
}

// Out-of-place window update: row j < new_len of every head of `out` is cache
// row shift + j for j < keep, else src row j - keep converted to the cache type.
// Each kept row crosses HBM once each way (the in-place form's two reversal
// passes move it twice), and the new rows land in the same launch. An item is
// 16 bytes of the cache side (E elements of TD); each thread moves two, items
// i and i + stride (stride = the launch's threads per head, so every memory
// instruction of a wave stays one contiguous run); grid.y walks the heads.
// Same-type moves copy raw bits. Measured on a one-token update of a full
// 8 x 8192 x 128 f16 cache (back-to-back launches): one item per thread
// 7.9 us, two 7.3 us, four 7.5 us; 512- or 1024-thread blocks and grid-stride
// loops over 1024-2048 blocks no faster; a device-to-device hipMemcpyAsync of
// the kept rows alone 8.0 us.
template <typename TS, typename TD, int E>
__global__ __launch_bounds__(kThreads) void kv_window_into(const TD* __restrict__ cache, const TS* __restrict__ src,
                                                           TD* __restrict__ out, uint32_t cpr, uint32_t keep,
                                                           uint32_t seq, uint64_t max_seq, uint64_t shift,
                                                           uint32_t items, uint64_t h0) {
    const uint32_t stride = gridDim.x * (uint32_t)kThreads;
    const uint32_t i0 = blockIdx.x * (uint32_t)kThreads + threadIdx.x;
    const uint64_t h = h0 + blockIdx.y;
    const uint64_t hd = (uint64_t)cpr * E;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const uint32_t i = i0 + (uint32_t)u * stride;
        if (i >= items) return;
        const uint32_t j = i / cpr;
        const uint32_t c = (i - j * cpr) * E;
        TD* d = out + (h * max_seq + j) * hd + c;
        if (j < keep) {
            const TD* s = cache + (h * max_seq + shift + j) * hd + c;
            vstore<true>(reinterpret_cast<u32x4*>(d), vload<true>(reinterpret_cast<const u32x4*>(s)));
        } else {
            move_chunk<TS, TD, E>(src + (h * seq + (j - keep)) * hd + c, d);
        }
    }
}

// Rows [shift, shift + keep) of every head of cache → rows [0, keep) of out,
// as raw units of UT (any row width: the Q8_0 cache's 34-byte blocks, odd
// head dims); the new rows are appended by a second launch.
template <typename UT>
__global__ __launch_bounds__(kThreads) void kv_copy_rows(const UT* __restrict__ cache, UT* __restrict__ out,
                                                         uint32_t units_per_row, uint64_t max_seq, uint64_t shift,
                                                         uint32_t items, uint64_t h0) {
    const uint32_t i = blockIdx.x * (uint32_t)kThreads + threadIdx.x;
    if (i >= items) return;
    const uint32_t j = i / units_per_row, u = i - j * units_per_row;
    const uint64_t base = (h0 + blockIdx.y) * max_seq * units_per_row + u;
    out[base + (uint64_t)j * units_per_row] = cache[base + (shift + j) * units_per_row];
}

constexpr uint64_t kMaxGridY = 65535;  // heads per launch

template <typename TS, typename TD>
int launch_window_into(const void* cache, const void* src, void* out, uint64_t n_heads, uint64_t hd, uint64_t seq,
                       uint64_t max_seq, uint64_t shift, uint64_t keep, hipStream_t stream) {
    constexpr int E = vec16<TD>::n;
    const uint64_t cpr = hd / E;
    const uint64_t items = (keep + seq) * cpr;
    const uint64_t threads = (items + 1) / 2;  // two items per thread
    for (uint64_t h0 = 0; h0 < n_heads; h0 += kMaxGridY) {
        const uint64_t nh = n_heads - h0 < kMaxGridY ? n_heads - h0 : kMaxGridY;
        const dim3 grid((unsigned)((threads + kThreads - 1) / kThreads), (unsigned)nh);
        const int st = launch(kv_window_into<TS, TD, E>, grid, kThreads, stream, static_cast<const TD*>(cache),
                              static_cast<const TS*>(src), static_cast<TD*>(out), (uint32_t)cpr, (uint32_t)keep,
                              (uint32_t)seq, max_seq, shift, (uint32_t)items, h0);
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

template <typename UT>
int launch_copy_rows(const void* cache, void* out, uint64_t n_heads, uint64_t row_bytes, uint64_t max_seq,
                     uint64_t shift, uint64_t keep, hipStream_t stream) {
    const uint64_t upr = row_bytes / sizeof(UT);
    const uint64_t items = keep * upr;
    if (items == 0) return SPH_OK;
    for (uint64_t h0 = 0; h0 < n_heads; h0 += kMaxGridY) {
        const uint64_t nh = n_heads - h0 < kMaxGridY ? n_heads - h0 : kMaxGridY;
        const dim3 grid((unsigned)((items + kThreads - 1) / kThreads), (unsigned)nh);
        const int st = launch(kv_copy_rows<UT>, grid, kThreads, stream, static_cast<const UT*>(cache),
                              static_cast<UT*>(out), (uint32_t)upr, max_seq, shift, (uint32_t)items, h0);
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

}  // namespace
}  // namespace sph

extern "C" int sph_transpose_heads(const void* x, void* out, int dtype, int64_t outer, int64_t inner,
                                   int64_t head_dim, void* stream) {
    if (outer < 0 || inner < 0 || head_dim < 0 || !sph::is_float_dtype(dtype)) return SPH_EINVAL;
    const uint64_t rows = (uint64_t)outer * (uint64_t)inner;
    if (rows == 0 || head_dim == 0) return SPH_OK;
    if (x == nullptr || out == nullptr || x == out) return SPH_EINVAL;
    if (outer > UINT32_MAX || inner > UINT32_MAX) return SPH_EINVAL;
    // The walk covers whole 8 x 8 tiles; padding rows are skipped in the kernel.
    const uint64_t t = sph::kTile;
    const uint64_t walk = (((uint64_t)outer + t - 1) / t) * (((uint64_t)inner + t - 1) / t) * t * t;
    const sph::RowMap m{(uint32_t)outer, (uint32_t)inner, 0};
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == SPH_F32) return sph::launch_move<float, float, sph::M_TRANSPOSE>(x, out, walk, head_dim, m, s);
    // Halves move as 16-bit patterns; the element type does not matter.
    return sph::launch_move<sph::f16, sph::f16, sph::M_TRANSPOSE>(x, out, walk, head_dim, m, s);
}

namespace {

// Every argument check of sph_kv_append: SPH_OK when the append would launch (or
// has nothing to do), else the error it returns. sph_kv_cache_update runs it
// before shifting, so a rejected call leaves the cache untouched.
int kv_append_check(const void* src, int src_dtype, const void* cache, int cache_dtype, int64_t n_kv, int64_t seq,
                    int64_t head_dim, int64_t max_seq, int64_t pos) {
    if (n_kv < 0 || seq < 0 || head_dim < 0 || max_seq < 0 || pos < 0) return SPH_EINVAL;
    const bool q8 = cache_dtype == SPH_Q8_0;
    if (!sph::is_float_dtype(src_dtype) || !(q8 || sph::is_float_dtype(cache_dtype))) return SPH_EINVAL;
    if (q8 && head_dim % 32 != 0) return SPH_EINVAL;
    if (pos > max_seq || seq > max_seq - pos) return SPH_ERANGE;
    const uint64_t rows = (uint64_t)n_kv * (uint64_t)seq;
    if (rows == 0 || head_dim == 0) return SPH_OK;
    if (src == nullptr || cache == nullptr) return SPH_EINVAL;
    if (seq > UINT32_MAX || max_seq > UINT32_MAX) return SPH_EINVAL;
    if (q8) {
        if (!sph::aligned(cache, 2) || !sph::aligned(src, 16) || head_dim / 32 > UINT32_MAX) return SPH_EINVAL;
        const uint64_t blocks = rows * ((uint64_t)head_dim / 32);
        if ((blocks + sph::kThreads - 1) / sph::kThreads > INT32_MAX) return SPH_EINVAL;
    } else if ((uint64_t)head_dim > (1u << 24) || rows > UINT32_MAX) {
        return SPH_EINVAL;  // launch_move's limits
    }
    return SPH_OK;
}

}  // namespace

extern "C" int sph_kv_append(const void* src, int src_dtype, void* cache, int cache_dtype, int64_t n_kv, int64_t seq,
                             int64_t head_dim, int64_t max_seq, int64_t pos, void* stream) {
    const int chk = kv_append_check(src, src_dtype, cache, cache_dtype, n_kv, seq, head_dim, max_seq, pos);
    if (chk != SPH_OK) return chk;
    const bool q8 = cache_dtype == SPH_Q8_0;
    const uint64_t rows = (uint64_t)n_kv * (uint64_t)seq;
    if (rows == 0 || head_dim == 0) return SPH_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (q8) {
        const uint64_t bpr = (uint64_t)head_dim / 32;
        const uint64_t blocks = rows * bpr;
        return sph::with_float_type(src_dtype, [&](auto ts) -> int {
            using TS = decltype(ts);
            const dim3 grid((unsigned)((blocks + sph::kThreads - 1) / sph::kThreads));
            return sph::launch(sph::kv_append_q8_0<TS>, grid, sph::kThreads, s, static_cast<const TS*>(src),
                               static_cast<uint8_t*>(cache), blocks, (uint32_t)bpr, (uint32_t)seq, (uint32_t)max_seq,
                               (uint64_t)pos);
        });
    }
    const sph::RowMap m{(uint32_t)seq, (uint32_t)max_seq, (uint64_t)pos};
    return sph::with_float_type(src_dtype, [&](auto ts) -> int {
        using TS = decltype(ts);
        return sph::with_float_type(cache_dtype, [&](auto td) -> int {
            using TD = decltype(td);
            return sph::launch_move<TS, TD, sph::M_KV>(src, cache, rows, head_dim, m, s);
        });
    });
}

extern "C" int sph_kv_cache_update(const void* src, int src_dtype, void* cache, int cache_dtype, int64_t n_kv,
                                   int64_t seq, int64_t head_dim, int64_t max_seq, int64_t cur_len, int64_t* new_len,
                                   void* stream) {
    if (n_kv < 0 || seq < 0 || head_dim < 0 || max_seq < 0 || cur_len < 0 || new_len == nullptr) return SPH_EINVAL;
    const bool q8 = cache_dtype == SPH_Q8_0;
    if (!sph::is_float_dtype(src_dtype) || !(q8 || sph::is_float_dtype(cache_dtype))) return SPH_EINVAL;
    if (q8 && head_dim % 32 != 0) return SPH_EINVAL;
    if (seq > max_seq) return SPH_ERANGE;      // the reference's "new tokens exceeds max cache size"
    if (cur_len > max_seq) return SPH_EINVAL;  // more valid rows than the cache holds
    const int64_t total = cur_len + seq;
    const int64_t shift = total > max_seq ? total - max_seq : 0;
    const int64_t keep = cur_len - shift;
    const int chk = kv_append_check(src, src_dtype, cache, cache_dtype, n_kv, seq, head_dim, max_seq, keep);
    if (chk != SPH_OK) return chk;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (shift > 0 && keep > 0 && n_kv > 0 && head_dim > 0) {
        if (cache == nullptr) return SPH_EINVAL;
        const uint64_t row_bytes = q8 ? (uint64_t)head_dim / 32 * 34 : (uint64_t)head_dim * sph::dtype_size(cache_dtype);
        int st;
        if (row_bytes % 16 == 0 && sph::aligned(cache, 16))
            st = sph::shift_window<sph::u32x4>(cache, n_kv, row_bytes, max_seq, shift, cur_len, s);
        else if (row_bytes % 8 == 0 && sph::aligned(cache, 8))
            st = sph::shift_window<sph::u32x2>(cache, n_kv, row_bytes, max_seq, shift, cur_len, s);
        else if (row_bytes % 4 == 0 && sph::aligned(cache, 4))
            st = sph::shift_window<uint32_t>(cache, n_kv, row_bytes, max_seq, shift, cur_len, s);
        else if (sph::aligned(cache, 2))
            st = sph::shift_window<uint16_t>(cache, n_kv, row_bytes, max_seq, shift, cur_len, s);
        else
            return SPH_EINVAL;
        if (st != SPH_OK) return st;
    }
    const int st = sph_kv_append(src, src_dtype, cache, cache_dtype, n_kv, seq, head_dim, max_seq, keep, stream);
    if (st != SPH_OK) return st;
    *new_len = total < max_seq ? total : max_seq;
    return SPH_OK;
}

namespace {

// [a, a + na) and [b, b + nb) share a byte.
bool overlaps(const void* a, uint64_t na, const void* b, uint64_t nb) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return na != 0 && nb != 0 && x < y + nb && y < x + na;
}

}  // namespace

extern "C" int sph_kv_cache_update_into(const void* src, int src_dtype, const void* cache, void* out, int cache_dtype,
                                        int64_t n_kv, int64_t seq, int64_t head_dim, int64_t max_seq,
                                        int64_t cur_len, int64_t* new_len, void* stream) {
    if (n_kv < 0 || seq < 0 || head_dim < 0 || max_seq < 0 || cur_len < 0 || new_len == nullptr) return SPH_EINVAL;
    const bool q8 = cache_dtype == SPH_Q8_0;
    if (!sph::is_float_dtype(src_dtype) || !(q8 || sph::is_float_dtype(cache_dtype))) return SPH_EINVAL;
    if (q8 && head_dim % 32 != 0) return SPH_EINVAL;
    if (seq > max_seq) return SPH_ERANGE;      // the reference's "new tokens exceeds max cache size"
    if (cur_len > max_seq) return SPH_EINVAL;  // more valid rows than the cache holds
    const int64_t total = cur_len + seq;
    const int64_t shift = total > max_seq ? total - max_seq : 0;
    const int64_t keep = cur_len - shift;
    const int64_t n_new = total < max_seq ? total : max_seq;
    // The append part's checks, against `out`.
    const int chk = kv_append_check(src, src_dtype, out, cache_dtype, n_kv, seq, head_dim, max_seq, keep);
    if (chk != SPH_OK) return chk;
    if (n_kv == 0 || head_dim == 0 || n_new == 0) {
        *new_len = n_new;
        return SPH_OK;
    }
    const uint64_t row_bytes = q8 ? (uint64_t)head_dim / 32 * 34 : (uint64_t)head_dim * sph::dtype_size(cache_dtype);
    const uint64_t cache_bytes = (uint64_t)n_kv * (uint64_t)max_seq * row_bytes;
    const uint64_t src_bytes = (uint64_t)n_kv * (uint64_t)seq * (uint64_t)head_dim * sph::dtype_size(src_dtype);
    if (out == nullptr || (keep > 0 && cache == nullptr)) return SPH_EINVAL;
    // out is written while cache and src are read.
    if ((keep > 0 && overlaps(cache, cache_bytes, out, cache_bytes)) || overlaps(src, src_bytes, out, cache_bytes))
        return SPH_EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);

    // Float caches whose rows split into 16-byte units: one launch does the move and the append.
    if (!q8 && sph::aligned(cache, 16) && sph::aligned(out, 16)) {
        const int64_t e = 16 / (int64_t)sph::dtype_size(cache_dtype);
        const uint64_t src_access = (uint64_t)e * sph::dtype_size(src_dtype);
        const uint64_t items = (uint64_t)n_new * (uint64_t)(head_dim / e);
        if (head_dim % e == 0 && sph::aligned(src, src_access < 16 ? src_access : 16) &&
            items <= UINT32_MAX - 2 * sph::kThreads) {  // i0 + stride stays below 2^32
            const int st = sph::with_float_type(src_dtype, [&](auto ts) -> int {
                using TS = decltype(ts);
                return sph::with_float_type(cache_dtype, [&](auto td) -> int {
                    using TD = decltype(td);
                    return sph::launch_window_into<TS, TD>(cache, src, out, n_kv, head_dim, seq, max_seq, shift,
                                                           keep, s);
                });
            });
            if (st != SPH_OK) return st;
            *new_len = n_new;
            return SPH_OK;
        }
    }
    // Any other row: the kept rows as raw units of the widest width both buffers allow, then the append.
    if (keep > 0) {
        auto fits = [&](uint64_t unit) {
            return row_bytes % unit == 0 && sph::aligned(cache, unit) && sph::aligned(out, unit) &&
                   row_bytes / unit <= UINT32_MAX && (uint64_t)keep * (row_bytes / unit) <= UINT32_MAX - sph::kThreads;
        };
        int st;
        if (fits(16)) st = sph::launch_copy_rows<sph::u32x4>(cache, out, n_kv, row_bytes, max_seq, shift, keep, s);
        else if (fits(8)) st = sph::launch_copy_rows<sph::u32x2>(cache, out, n_kv, row_bytes, max_seq, shift, keep, s);
        else if (fits(4)) st = sph::launch_copy_rows<uint32_t>(cache, out, n_kv, row_bytes, max_seq, shift, keep, s);
        else if (fits(2)) st = sph::launch_copy_rows<uint16_t>(cache, out, n_kv, row_bytes, max_seq, shift, keep, s);
        else return SPH_EINVAL;
        if (st != SPH_OK) return st;
    }
    const int st = sph_kv_append(src, src_dtype, out, cache_dtype, n_kv, seq, head_dim, max_seq, keep, stream);
    if (st != SPH_OK) return st;
    *new_len = n_new;
    return SPH_OK;
}
