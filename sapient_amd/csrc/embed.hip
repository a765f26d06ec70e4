// embed.hip — token-embedding gather with in-register GGUF row dequantization, gfx950.
//
// Reference: common::embed_tokens → gather_row_f32
// (crates/sapient-models/src/forward/common.rs:164-217) and the dequant arms of
// Tensor::to_f32_vec (crates/sapient-core/src/tensor.rs:362-398, Q4_K
// :504-527 with get_scale_min_k4 :567-576, Q5_K :421-467, Q6_K :534-565):
//   Q4_0 (18-byte block of 32): y = f32(q − 8) · f32(d), q the low nibbles of
//        bytes 0..15 for elements 0..15 and their high nibbles for 16..31
//   Q8_0 (34-byte block of 32): y = f32(i8 q) · f32(d)
//   Q4_K (144-byte block of 256): y = (d·sc)·q − dmin·m, 6-bit (sc, m) unpacked per
//        32-element sub-block, low nibbles then high nibbles per 64 elements
//   Q5_K (176-byte block of 256): as Q4_K with q + 16·h, h one bit per element
//        from the 32-byte qh plane (bit 2c of qh[l] for the low-nibble half of
//        64-element chunk c, bit 2c + 1 for the high-nibble half)
//   Q6_K (210-byte block of 256): y = (d·sc)·(q − 32)
// Every product above is exact in f32 (≤ 22 significant bits) except Q6_K's
// last one, which is rounded in the reference's order; the K-quants' single
// rounding is the final subtraction, which one FMA performs identically
// (d·sc·q is exact). The gather is therefore bit-exact.
//
// Design (write-dominated: 16 KiB of f32 out per 2.3 KiB Q4_K row in):
//  - One wave64 per token (16 tokens per 1024-thread block; 8 per 512-thread
//    block in embed_staged, whose LDS footprint that keeps small, and 2 per
//    block when there are too few ids to give every CU a block); each lane produces
//    4 consecutive outputs per step, so every store instruction writes 1 KiB
//    contiguous (16 bytes per lane), non-temporal (non-temporal stores and the
//    larger block measured 4.8 → 6.5 TB/s on the Q4_K gather).
//  - The packed blocks are consumed as stored — no repacking. A wave first
//    copies its row (a chunk of whole blocks at a time) into LDS with the
//    widest loads the row length and table address allow (16, 8 or 4 bytes),
//    each cache line requested by one lane and a chunk's loads all in flight
//    together, then dequantizes from LDS (embed_staged; Q4_K: embed_q4_k_staged,
//    which takes one 256-element super-block per step: a lane reads the
//    16-byte header (d, dmin, 12 scale bytes) and the dword of nibbles it needs
//    and unpacks its (sc, m) pair in registers).
//  - Rows whose length or address admits only 2-byte loads (Q4_0, Q8_0 and
//    Q6_K blocks are 18, 34 and 210 bytes) are read in place (embed_rows).
//  - An id >= vocab zero-fills its row and raises `bad_id_flag`; the table is
//    never read out of bounds.
#include <type_traits>

#include "sph_common.h"

namespace sph {
namespace {

constexpr int kThreads = 1024;
constexpr int kWave = 64;
constexpr int kTokPerBlock = kThreads / kWave;

__device__ __forceinline__ float f16_at(const uint8_t* p) {
    return widen(f16{*reinterpret_cast<const uint16_t*>(p)});
}

// Output rows are written once and not re-read by this kernel: non-temporal.
__device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
    f32x4 v = {a, b, c, d};
    vstore<true>(reinterpret_cast<f32x4*>(p), v);
}

// Dequantize elements [4e, 4e + 4) of one row into `o`.
template <int DT>
__device__ __forceinline__ void dequant4(const uint8_t* __restrict__ row, int e4, float (&o)[4]);

template <>
__device__ __forceinline__ void dequant4<SPH_F32>(const uint8_t* __restrict__ row, int e4, float (&o)[4]) {
    const f32x4 v = reinterpret_cast<const f32x4*>(row)[e4];
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
}

template <>
__device__ __forceinline__ void dequant4<SPH_F16>(const uint8_t* __restrict__ row, int e4, float (&o)[4]) {
    const u32x2 v = reinterpret_cast<const u32x2*>(row)[e4];
    o[0] = widen(f16{(uint16_t)v.x}); o[1] = widen(f16{(uint16_t)(v.x >> 16)});
    o[2] = widen(f16{(uint16_t)v.y}); o[3] = widen(f16{(uint16_t)(v.y >> 16)});
}

template <>
__device__ __forceinline__ void dequant4<SPH_BF16>(const uint8_t* __restrict__ row, int e4, float (&o)[4]) {
    const u32x2 v = reinterpret_cast<const u32x2*>(row)[e4];
    o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xFFFF0000u);
    o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xFFFF0000u);
}

template <>
__device__ __forceinline__ void dequant4<SPH_Q8_0>(const uint8_t* __restrict__ row, int e4, float (&o)[4]) {
    const int blk = e4 >> 3;            // 8 groups of 4 per 32-element block
    const int j = (e4 & 7) * 4;
    const uint8_t* b = row + blk * 34;
    const float d = f16_at(b);
    const uint16_t* q = reinterpret_cast<const uint16_t*>(b + 2 + j);  // 2-byte aligned
    const uint32_t lo = q[0], hi = q[1];
    o[0] = (float)(int8_t)(lo & 0xFF) * d;
    o[1] = (float)(int8_t)(lo >> 8) * d;
    o[2] = (float)(int8_t)(hi & 0xFF) * d;
    o[3] = (float)(int8_t)(hi >> 8) * d;
}

template <>
__device__ __forceinline__ void dequant4<SPH_Q4_0>(const uint8_t* __restrict__ row, int e4, float (&o)[4]) {
    const int blk = e4 >> 3;            // 8 groups of 4 per 32-element block
    const int j = (e4 & 7) * 4;         // first element of the group
    const uint8_t* b = row + blk * 18;
    const float d = f16_at(b);
    const uint16_t* q = reinterpret_cast<const uint16_t*>(b + 2 + (j & 15));  // 2-byte aligned
    const uint32_t w = (uint32_t)q[0] | ((uint32_t)q[1] << 16);
    const int sh = j >= 16 ? 4 : 0;     // elements 16..31 are the high nibbles
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = (float)((int)((w >> (8 * c + sh)) & 0xF) - 8) * d;
}

// 6-bit (sc, m) of sub-block sb (0..7) from the 12 scale bytes of a K-quant
// header whose dwords 1..3 are s0, s1, s2 (get_scale_min_k4, tensor.rs:567-576).
__device__ __forceinline__ void scale_min_k4(uint32_t s0, uint32_t s1, uint32_t s2, int sb, uint32_t& sc,
                                             uint32_t& m) {
    const int sh = 8 * (sb & 3);
    const uint32_t A = (s0 >> sh) & 0xFF;  // scales[sb & 3]
    const uint32_t B = (s1 >> sh) & 0xFF;  // scales[(sb & 3) + 4]
    const uint32_t C = (s2 >> sh) & 0xFF;  // scales[(sb & 3) + 8]
    if (sb < 4) {
        sc = A & 63;
        m = B & 63;
    } else {
        sc = (C & 0x0F) | ((A >> 6) << 4);
        m = (C >> 4) | ((B >> 6) << 4);
    }
}

template <>
__device__ __forceinline__ void dequant4<SPH_Q5_K>(const uint8_t* __restrict__ row, int e4, float (&o)[4]) {
    const int blk = e4 >> 6;            // 64 groups of 4 per 256-element super-block
    const int e = (e4 & 63) * 4;        // element within the super-block
    const int c = e >> 6;               // 64-element chunk 0..3
    const int hi = (e >> 5) & 1;        // 0: low nibbles, 1: high nibbles of the chunk's 32 bytes
    const int l = e & 31;               // 4 consecutive l
    const uint8_t* b = row + blk * 176;  // 16-byte aligned
    const u32x4 hdr = *reinterpret_cast<const u32x4*>(b);
    const uint32_t qh = *reinterpret_cast<const uint32_t*>(b + 16 + l);
    const uint32_t ql = *reinterpret_cast<const uint32_t*>(b + 48 + 32 * c + l);
    uint32_t sc, m;
    scale_min_k4(hdr.y, hdr.z, hdr.w, 2 * c + hi, sc, m);
    const float d1 = widen(f16{(uint16_t)hdr.x}) * (float)sc;
    const float m1 = widen(f16{(uint16_t)(hdr.x >> 16)}) * (float)m;
    const int plane = 2 * c + hi;       // the qh bit of this half-chunk
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t q = ((ql >> (8 * k + 4 * hi)) & 0xF) | (((qh >> (8 * k + plane)) & 1u) << 4);
        o[k] = __builtin_fmaf(d1, (float)q, -m1);
    }
}

template <>
__device__ __forceinline__ void dequant4<SPH_Q6_K>(const uint8_t* __restrict__ row, int e4, float (&o)[4]) {
    const int blk = e4 >> 6;            // 64 groups of 4 per 256-element super-block
    const int e = (e4 & 63) * 4;        // element within the super-block
    const int n = e >> 7;               // 128-element half
    const int g = (e & 127) >> 5;       // quarter within the half (0..3)
    const int l = e & 31;               // 4 consecutive l
    const uint8_t* b = row + blk * 210;
    const float d = f16_at(b + 208);
    const uint16_t* ql = reinterpret_cast<const uint16_t*>(b + 64 * n + 32 * (g & 1) + l);
    const uint16_t* qh = reinterpret_cast<const uint16_t*>(b + 128 + 32 * n + l);
    const uint32_t qlw = (uint32_t)ql[0] | ((uint32_t)ql[1] << 16);
    const uint32_t qhw = (uint32_t)qh[0] | ((uint32_t)qh[1] << 16);
    const float dsc = d * (float)(int8_t)b[192 + 8 * n + (l >> 4) + 2 * g];
    const int lshift = (g >> 1) * 4;    // quarters 2, 3 use the high nibbles
    const int hshift = 2 * g;           // qh bits 2g..2g+1
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int ql4 = (qlw >> (8 * c + lshift)) & 0xF;
        const int qh2 = (qhw >> (8 * c + hshift)) & 0x3;
        o[c] = dsc * (float)((ql4 | (qh2 << 4)) - 32);
    }
}

// Q4_K: a lane handles elements [4l, 4l + 4) of a super-block, l = lane.
// `hdr` is the block's first 16 bytes (d, dmin, scales[0..12)), `qw` the
// dword of nibbles this lane needs.
__device__ __forceinline__ void dequant_q4k_lane(const u32x4 hdr, uint32_t qw, int lane, float (&o)[4]) {
    const int sb = lane >> 3;            // 32-element sub-block 0..7
    const float d = widen(f16{(uint16_t)hdr.x});
    const float dmin = widen(f16{(uint16_t)(hdr.x >> 16)});
    uint32_t sc, m;
    scale_min_k4(hdr.y, hdr.z, hdr.w, sb, sc, m);
    const float d1 = d * (float)sc;
    const float m1 = dmin * (float)m;
    const uint32_t nib = (sb & 1) ? (qw >> 4) & 0x0F0F0F0Fu : qw & 0x0F0F0F0Fu;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = __builtin_fmaf(d1, (float)((nib >> (8 * c)) & 0xFF), -m1);
}

template <int DT>
__global__ __launch_bounds__(kThreads) void embed_rows(const uint8_t* __restrict__ table, int64_t vocab,
                                                       int hidden, int64_t row_bytes, const uint32_t* __restrict__ ids,
                                                       int64_t n_ids, float* __restrict__ out, int32_t* bad_id_flag) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t t = (int64_t)blockIdx.x * kTokPerBlock + (threadIdx.x / kWave);
    if (t >= n_ids) return;
    // The token is wave-uniform: broadcast its id so the row base (and every
    // block header address) lives in scalar registers.
    const uint32_t id = __builtin_amdgcn_readfirstlane(ids[t]);
    float* dst = out + (size_t)t * (size_t)hidden;
    const int n4 = hidden / 4;
    if ((int64_t)id >= vocab) {
        for (int e4 = lane; e4 < n4; e4 += kWave) store4(dst + 4 * e4, 0.f, 0.f, 0.f, 0.f);
        if (lane == 0 && bad_id_flag != nullptr) *bad_id_flag = 1;
        return;
    }
    const uint8_t* row = table + (size_t)id * (size_t)row_bytes;
    for (int e4 = lane; e4 < n4; e4 += kWave) {
        float o[4];
        dequant4<DT>(row, e4, o);
        store4(dst + 4 * e4, o[0], o[1], o[2], o[3]);
    }
}

// Rows staged through LDS (every table type but Q4_K, which has its own lane
// mapping below). Reading blocks in place waits on memory once per step of
// four outputs per lane: at 65536 random ids of a 128256 x 4096 table whose
// rows come from HBM, Q4_0 / Q5_K / Q6_K in place ran at 54-60 % of HBM peak.
// A wave instead copies a chunk of its row (whole blocks, at most kStageBytes)
// into LDS with W-byte loads — W the widest power of two dividing both the row
// length and the table's alignment, so every line is requested once and all of
// a chunk's loads are in flight together — and dequantizes from there with
// the same per-element arithmetic as embed_rows. Every wave of a block runs
// the same number of chunk steps (hidden is uniform), so the block barriers
// are reached by all, tokens past n_ids included.
// Blocks of 8 waves (512 threads) x 4608 B: four blocks fit a CU's LDS, and
// against 16-wave blocks (two per CU) they measured 0.6 to 1.9 points more of
// HBM peak on every staged type at 65536 uniform ids of a 128256 x 4096 table
// (Q5_K 75.8 -> 76.5 %, Q8_0 74.8 -> 75.6 %, f16 73.0 -> 74.9 %). The Q4_K
// kernel below stages 2304 B per wave and gains nothing from the smaller block.
constexpr int kStageBytes = 4608;
constexpr int kStagedThreads = 512;
constexpr int kStagedTokPerBlock = kStagedThreads / kWave;
constexpr int kFewTokPerBlock = 2;

template <int W> struct StageWord;
template <> struct StageWord<16> { using type = u32x4; };
template <> struct StageWord<8> { using type = u32x2; };
template <> struct StageWord<4> { using type = uint32_t; };

// Bytes and elements of the unit a staged chunk is cut in: a quantization
// block, or four elements of a plain table (hidden is a multiple of 4).
template <int DT> struct StageUnit;
template <> struct StageUnit<SPH_F32> { static constexpr int bytes = 16, elems = 4; };
template <> struct StageUnit<SPH_F16> { static constexpr int bytes = 8, elems = 4; };
template <> struct StageUnit<SPH_BF16> { static constexpr int bytes = 8, elems = 4; };
template <> struct StageUnit<SPH_Q4_0> { static constexpr int bytes = 18, elems = 32; };
template <> struct StageUnit<SPH_Q8_0> { static constexpr int bytes = 34, elems = 32; };
template <> struct StageUnit<SPH_Q5_K> { static constexpr int bytes = 176, elems = 256; };
template <> struct StageUnit<SPH_Q6_K> { static constexpr int bytes = 210, elems = 256; };

// chunk_units: units per chunk, chunk_units * bytes <= kStageBytes and a multiple of W.
// TPB: tokens (waves) per block.
template <int DT, int W, int TPB>
__global__ __launch_bounds__(TPB * kWave) void embed_staged(const uint8_t* __restrict__ table, int64_t vocab, int hidden,
                                                      int64_t row_bytes, const uint32_t* __restrict__ ids,
                                                      int64_t n_ids, float* __restrict__ out, int32_t* bad_id_flag,
                                                      int chunk_units) {
    using Word = typename StageWord<W>::type;
    using U = StageUnit<DT>;
    __shared__ __align__(16) uint8_t stage[TPB][kStageBytes];
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave;
    const int64_t t = (int64_t)blockIdx.x * TPB + wv;
    const bool active = t < n_ids;
    const uint32_t id = active ? __builtin_amdgcn_readfirstlane(ids[t]) : 0u;
    const bool valid = active && (int64_t)id < vocab;
    float* dst = out + (size_t)(active ? t : 0) * (size_t)hidden;
    if (active && !valid) {
        for (int e4 = lane; e4 < hidden / 4; e4 += kWave) store4(dst + 4 * e4, 0.f, 0.f, 0.f, 0.f);
        if (lane == 0 && bad_id_flag != nullptr) *bad_id_flag = 1;
    }
    const uint8_t* row = table + (size_t)(valid ? id : 0u) * (size_t)row_bytes;
    uint8_t* buf = stage[wv];
    const int nunits = hidden / U::elems;
    for (int c0 = 0; c0 < nunits; c0 += chunk_units) {
        const int nu = nunits - c0 < chunk_units ? nunits - c0 : chunk_units;
        const int bytes = nu * U::bytes;  // a multiple of W: so are row_bytes and chunk_units * U::bytes
        if (valid) {
            const uint8_t* src = row + (size_t)c0 * U::bytes;
            for (int o = lane * W; o < bytes; o += kWave * W)
                *reinterpret_cast<Word*>(buf + o) = *reinterpret_cast<const Word*>(src + o);
        }
        __syncthreads();
        if (valid) {
            float* d0 = dst + (size_t)c0 * U::elems;
            for (int e4 = lane; e4 < nu * (U::elems / 4); e4 += kWave) {
                float o[4];
                dequant4<DT>(buf, e4, o);
                store4(d0 + 4 * e4, o[0], o[1], o[2], o[3]);
            }
        }
        __syncthreads();
    }
}

// Q4_K rows staged through LDS: a 144-byte super-block spans two cache lines,
// one of them shared with its neighbour, and per-block loads fetched ~35 % of
// each row twice (rocprofv3 FETCH_SIZE at 65536 uniform ids of a 128256 x
// 4096 table: 1.35x the row bytes). A wave instead copies up to
// kQ4kChunkBlocks super-blocks of its row into LDS with 16-byte loads (every
// line requested once, by one lane) and dequantizes from there with the same
// per-lane arithmetic as embed_rows. Every wave of a block runs the same
// number of chunk steps, so the block barriers are reached by all.
constexpr int kQ4kChunkBlocks = 16;
constexpr int kQ4kChunkBytes = kQ4kChunkBlocks * 144;  // a multiple of 16

__global__ __launch_bounds__(kThreads) void embed_q4_k_staged(const uint8_t* __restrict__ table, int64_t vocab,
                                                              int hidden, int64_t row_bytes,
                                                              const uint32_t* __restrict__ ids, int64_t n_ids,
                                                              float* __restrict__ out, int32_t* bad_id_flag) {
    __shared__ __align__(16) uint8_t stage[kTokPerBlock][kQ4kChunkBytes];
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave;
    const int64_t t = (int64_t)blockIdx.x * kTokPerBlock + wv;
    const bool active = t < n_ids;
    const uint32_t id = active ? __builtin_amdgcn_readfirstlane(ids[t]) : 0u;
    const bool valid = active && (int64_t)id < vocab;
    float* dst = out + (size_t)(active ? t : 0) * (size_t)hidden;
    if (active && !valid) {
        for (int e4 = lane; e4 < hidden / 4; e4 += kWave) store4(dst + 4 * e4, 0.f, 0.f, 0.f, 0.f);
        if (lane == 0 && bad_id_flag != nullptr) *bad_id_flag = 1;
    }
    const uint8_t* row = table + (size_t)(valid ? id : 0u) * (size_t)row_bytes;
    uint8_t* buf = stage[wv];
    const int nblk = hidden / 256;
    const int qoff = 16 + 32 * (lane >> 4) + 4 * (lane & 7);  // this lane's nibble dword in a block
    for (int c0 = 0; c0 < nblk; c0 += kQ4kChunkBlocks) {
        const int nb = nblk - c0 < kQ4kChunkBlocks ? nblk - c0 : kQ4kChunkBlocks;
        if (valid) {
            const uint8_t* src = row + (size_t)c0 * 144;
            for (int o = lane * 16; o < nb * 144; o += kWave * 16)
                *reinterpret_cast<u32x4*>(buf + o) = *reinterpret_cast<const u32x4*>(src + o);
        }
        __syncthreads();
        if (valid) {
            for (int j = 0; j < nb; ++j) {
                const uint8_t* b = buf + j * 144;
                float o[4];
                dequant_q4k_lane(*reinterpret_cast<const u32x4*>(b), *reinterpret_cast<const uint32_t*>(b + qoff),
                                 lane, o);
                store4(dst + 256 * (c0 + j) + 4 * lane, o[0], o[1], o[2], o[3]);
            }
        }
        __syncthreads();
    }
}

int launch_q4_k_staged(const void* table, int64_t vocab, int64_t hidden, int64_t row_bytes, const uint32_t* ids,
                       int64_t n_ids, float* out, int32_t* flag, hipStream_t stream) {
    constexpr int64_t kChunk = int64_t(1) << 24;  // tokens per launch
    for (int64_t t0 = 0; t0 < n_ids; t0 += kChunk) {
        const int64_t nt = n_ids - t0 < kChunk ? n_ids - t0 : kChunk;
        const dim3 grid((unsigned)((nt + kTokPerBlock - 1) / kTokPerBlock));
        const int st = launch(embed_q4_k_staged, grid, kThreads, stream, static_cast<const uint8_t*>(table), vocab,
                              (int)hidden, row_bytes, ids + t0, nt, out + (size_t)t0 * (size_t)hidden, flag);
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

// Units per staged chunk: as many as fit kStageBytes with chunk bytes a multiple of W
// (W / gcd(unit bytes, W) <= 16 units always qualify and fit).
template <int DT>
int stage_chunk_units(int W) {
    int cu = kStageBytes / StageUnit<DT>::bytes;
    while (cu > 1 && (cu * StageUnit<DT>::bytes) % W != 0) --cu;
    return cu;
}

template <int DT, int W>
int launch_staged(const void* table, int64_t vocab, int64_t hidden, int64_t row_bytes, const uint32_t* ids,
                  int64_t n_ids, float* out, int32_t* flag, hipStream_t stream) {
    const int cu = stage_chunk_units<DT>(W);
    if ((cu * StageUnit<DT>::bytes) % W != 0 || row_bytes % W != 0) return SPH_EINVAL;
    constexpr int64_t kChunk = int64_t(1) << 24;  // tokens per launch
    for (int64_t t0 = 0; t0 < n_ids; t0 += kChunk) {
        const int64_t nt = n_ids - t0 < kChunk ? n_ids - t0 : kChunk;
        // Too few ids for one 8-wave block per CU (a decode step, a prefill chunk): 2-wave
        // blocks, four times as many CUs. Per launch, back to back on MI355X: Q8_0 151936 x 896,
        // 512 ids 2.49 -> 2.38-2.42 µs; F16 51200 x 2560, 64 ids 3.22 -> 2.93, 512 ids 3.57 ->
        // 3.17-3.29 (one and four waves per block measured between the two).
        if (nt <= (int64_t)kStagedTokPerBlock * device_cu_count()) {
            const dim3 g2((unsigned)((nt + kFewTokPerBlock - 1) / kFewTokPerBlock));
            const int st2 = launch(embed_staged<DT, W, kFewTokPerBlock>, g2, kFewTokPerBlock * kWave, stream,
                                   static_cast<const uint8_t*>(table), vocab, (int)hidden, row_bytes, ids + t0, nt,
                                   out + (size_t)t0 * (size_t)hidden, flag, cu);
            if (st2 != SPH_OK) return st2;
            continue;
        }
        const dim3 grid((unsigned)((nt + kStagedTokPerBlock - 1) / kStagedTokPerBlock));
        const int st = launch(embed_staged<DT, W, kStagedTokPerBlock>, grid, kStagedThreads, stream, static_cast<const uint8_t*>(table), vocab,
                              (int)hidden, row_bytes, ids + t0, nt, out + (size_t)t0 * (size_t)hidden, flag, cu);
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

template <int DT>
int launch_embed(const void* table, int64_t vocab, int64_t hidden, int64_t row_bytes, const uint32_t* ids,
                 int64_t n_ids, float* out, int32_t* flag, hipStream_t stream) {
    constexpr int64_t kChunk = int64_t(1) << 24;  // tokens per launch
    for (int64_t t0 = 0; t0 < n_ids; t0 += kChunk) {
        const int64_t nt = n_ids - t0 < kChunk ? n_ids - t0 : kChunk;
        const dim3 grid((unsigned)((nt + kTokPerBlock - 1) / kTokPerBlock));
        const int st = launch(embed_rows<DT>, grid, kThreads, stream, static_cast<const uint8_t*>(table), vocab,
                              (int)hidden, row_bytes, ids + t0, nt, out + (size_t)t0 * (size_t)hidden, flag);
        if (st != SPH_OK) return st;
    }
    return SPH_OK;
}

}  // namespace
}  // namespace sph

extern "C" int sph_embed(const void* table, int table_dtype, int64_t vocab, int64_t hidden, const uint32_t* ids,
                         int64_t n_ids, float* out, int32_t* bad_id_flag, void* stream) {
    using namespace sph;
    if (vocab < 0 || hidden <= 0 || n_ids < 0 || hidden > INT32_MAX / 4) return SPH_EINVAL;
    int64_t row_bytes = 0;
    size_t align = 16;
    switch (table_dtype) {
    case SPH_F32: row_bytes = hidden * 4; if (hidden % 4) return SPH_EINVAL; break;
    case SPH_F16:
    case SPH_BF16: row_bytes = hidden * 2; align = 8; if (hidden % 4) return SPH_EINVAL; break;
    case SPH_Q4_0: if (hidden % 32) return SPH_EINVAL; row_bytes = hidden / 32 * 18; align = 2; break;
    case SPH_Q8_0: if (hidden % 32) return SPH_EINVAL; row_bytes = hidden / 32 * 34; align = 2; break;
    case SPH_Q4_K: if (hidden % 256) return SPH_EINVAL; row_bytes = hidden / 256 * 144; break;
    case SPH_Q5_K: if (hidden % 256) return SPH_EINVAL; row_bytes = hidden / 256 * 176; break;
    case SPH_Q6_K: if (hidden % 256) return SPH_EINVAL; row_bytes = hidden / 256 * 210; align = 2; break;
    default: return SPH_EINVAL;
    }
    if (n_ids == 0) return SPH_OK;
    if (ids == nullptr || out == nullptr || (vocab > 0 && table == nullptr)) return SPH_EINVAL;
    if (!aligned(table, align) || !aligned(out, 16) || !aligned(ids, 4)) return SPH_EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (table_dtype == SPH_Q4_K)
        return launch_q4_k_staged(table, vocab, hidden, row_bytes, ids, n_ids, out, bad_id_flag, s);
    // Every other type: staged through LDS with the widest loads the row length and table
    // address allow, or read in place when only 2-byte loads would do.
    const int W = (row_bytes % 16 == 0 && aligned(table, 16)) ? 16
                : (row_bytes % 8 == 0 && aligned(table, 8))   ? 8
                : (row_bytes % 4 == 0 && aligned(table, 4))   ? 4 : 0;
    auto go = [&](auto dt) -> int {
        constexpr int DT = decltype(dt)::value;
        switch (W) {
        case 16: return launch_staged<DT, 16>(table, vocab, hidden, row_bytes, ids, n_ids, out, bad_id_flag, s);
        case 8: return launch_staged<DT, 8>(table, vocab, hidden, row_bytes, ids, n_ids, out, bad_id_flag, s);
        case 4: return launch_staged<DT, 4>(table, vocab, hidden, row_bytes, ids, n_ids, out, bad_id_flag, s);
        default: return launch_embed<DT>(table, vocab, hidden, row_bytes, ids, n_ids, out, bad_id_flag, s);
        }
    };
    switch (table_dtype) {
    case SPH_F32: return go(std::integral_constant<int, SPH_F32>{});
    case SPH_F16: return go(std::integral_constant<int, SPH_F16>{});
    case SPH_BF16: return go(std::integral_constant<int, SPH_BF16>{});
    case SPH_Q4_0: return go(std::integral_constant<int, SPH_Q4_0>{});
    case SPH_Q8_0: return go(std::integral_constant<int, SPH_Q8_0>{});
    case SPH_Q5_K: return go(std::integral_constant<int, SPH_Q5_K>{});
    case SPH_Q6_K: return go(std::integral_constant<int, SPH_Q6_K>{});
    }
    return SPH_EINVAL;
}
