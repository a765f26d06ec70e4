// rope.hip — rotary position embedding (NEOX and interleaved), in place, gfx950.
//
// Reference math (crates/sapient-backends/cpu/src/kernels/rope.rs:48-57, :123-129):
//   freq = (pos as f32 / pos_scale) / powf(base, 2i / rotary_dim)
//   o[a] = x[a]·cos(freq) − x[b]·sin(freq);   o[b] = x[b]·cos(freq) + x[a]·sin(freq)
// with (a, b) = (i, i + rotary_dim/2) for NEOX and (2i, 2i + 1) for the
// interleaved layout (gguf_weights.rs:111-115 defines the permutation between them).
//
// Design:
//  - A thread owns P consecutive pairs (i0 .. i0+P) of one token and walks a
//    group of heads of Q and K: sin/cos are computed once per (position, pair)
//    and reused for every head (40 at the Llama-3-8B shape), so the
//    transcendental cost is amortised and the loop over heads is pure
//    16-byte load / FMA-free arithmetic / 16-byte store, non-temporal (each
//    element is read once and written once).
//  - Parity: the d/2 denominators powf(base, 2i/d) come from the host's libm
//    (the call the reference makes, passed in as kernel arguments); the
//    division by them is IEEE f32 in-kernel; sin and cos are glibc's sinf and
//    cosf restated (glibc_sincosf.h, bit-exact with the host libm over every
//    f32 input); the rotation rounds each product before the add/subtract
//    (-ffp-contract=off), exactly as the reference. The result is therefore
//    the reference's, bit for bit.
//  - grid.x covers tokens, grid.y splits the heads into groups (512-1024
//    blocks in all) so that short sequences still put waves on every CU.
//  - The decode-step variant (sph_rope_kv_append) fuses the RoPE of q and k
//    with the KV-cache append of k and v (resident.rs:467 then :645-711): the
//    same threads that rotate a k row write it, and the matching v row, into
//    the caches at the position read from device memory, converted to the
//    cache type. One launch instead of three, and since no host-side position
//    is baked into its arguments, a captured HIP graph replays it token after
//    token.
#include <math.h>

#include <type_traits>

#include "glibc_sincosf.h"
#include "sph_common.h"
#include "sph_internal.h"

namespace sph {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxHalf = 256;  // rotary_dim <= 512

struct DenTable {
    float v[kMaxHalf];
};

// Angles read from caller-supplied tables instead of evaluated: row r of cs /
// sn holds cos / sin of position r's angle for pairs 0 .. half - 1 (the layout
// of rope_cos_sin_cache, crates/sapient-backends/cpu/src/kernels/rope.rs:140-153).
// Token s reads row pos[s] (row s when pos is null); a row outside [0, rows)
// leaves the token's channels unchanged and stores 1 to *bad (when not null).
struct TableArgs {
    const float* cs;
    const float* sn;
    int64_t rows;
    int32_t* bad;
};

__constant__ InvPio4Table kInvPio4 = inv_pio4_table();

// The large-argument reduction indexes the 4/pi table per lane; staged in LDS
// the lookups stay off the vector-memory queue the row stream keeps full
// (measured: ~1.5 µs of 58 at the Llama-3-8B shape). Every thread of the block
// must call this before any returns.
__device__ __forceinline__ const uint32_t* stage_inv_pio4(uint32_t (&tab)[24]) {
    if (threadIdx.x < 24) tab[threadIdx.x] = kInvPio4.w[threadIdx.x];
    __syncthreads();
    return tab;
}

// L consecutive elements of one row held as they sit in memory (32-bit words,
// or single elements when the run is narrower than a word or ELEM asks for
// element accesses: rows only element-aligned), so that a batch of rows can be
// in flight while the previous batch is rotated and stored.
template <typename T, int L, bool ELEM = false>
struct RawRun {
    static constexpr bool kWords = !ELEM && (L * (int)sizeof(T)) % 4 == 0;
    uint32_t w[kWords ? words_of<T, L>::n : 1];
    T e[kWords ? 1 : L];

    __device__ __forceinline__ void load(const T* p) {
        if constexpr (kWords) {
            load_words<T, L, true>(p, w);
        } else {
#pragma unroll
            for (int i = 0; i < L; ++i) e[i] = p[i];
        }
    }
    __device__ __forceinline__ void to_f32(float (&v)[L]) const {
        if constexpr (kWords) {
            words_to_f32<T, L>(w, v);
        } else {
#pragma unroll
            for (int i = 0; i < L; ++i) v[i] = widen(e[i]);
        }
    }
};

template <typename T, int L, bool ELEM = false>
__device__ __forceinline__ void store_run(T* p, const float (&v)[L]) {
    if constexpr (!ELEM && (L * (int)sizeof(T)) % 4 == 0) {
        store_f32<T, L, true>(p, v);
    } else {
#pragma unroll
        for (int i = 0; i < L; ++i) p[i] = narrow<T>(v[i]);
    }
}

// One thread: pairs of one token, over the heads [h_begin, h_end) of its
// group, U heads per batch. Each row is read as R runs of L elements:
//  - NEOX: runs of P at i0 and i0 + half, rotating pairs (i0 + j, i0 + half + j);
//  - interleaved: one run of 2P at 2·i0, pairs i0 .. i0 + P;
//  - interleaved, SPLIT: runs of 2P at 2·i0 and 2·i0 + half, pairs i0 .. i0 + P
//    and i0 + half/2 .. i0 + half/2 + P — two requests per head like NEOX,
//    which streams faster than one request of twice the size (f32 at the
//    Llama-3-8B shape: 61.2 µs with one 16-byte run per thread, 58.0 µs split).
// NA = the distinct angles a thread applies (P, or 2P when SPLIT). kPre
// batches of U heads are requested before the angles are computed, so the
// angle phase overlaps their loads; from then on one batch is in flight while
// the other is rotated and stored. The half types request four (eight heads:
// f16 at the Llama-3-8B shape, NEOX 30.2 -> 28.4 us, interleaved 30.0 ->
// 28.4, the speed of the same access pattern with no arithmetic at all;
// three: 29.5 / 29.0; five need more than 64 VGPRs, lose half the resident
// waves and run at 33.2). In steady state two stay best: more requests in
// flight per wave slowed every stream measured on this GPU.
//
// PAIR_MAJOR: angles are computed pair-major over the block (slot j of
// thread x takes angle j·blockDim + x of the [pair][token] order), not per
// thread: the lanes of a wave then hold a few adjacent pairs, all with similar
// angles, and only the waves whose pairs are low enough to see |angle| >= 120
// (at long sequences, the first ~20 of 64 pairs) run glibc's large-argument
// reduction. Per-thread angles (pairs i0 .. i0+P of one token) put low pairs
// in every wave, which made every wave pay for both reductions. sin and cos
// reach the threads that apply them through LDS. Measured at 32 + 8 heads x
// 8192 tokens x 128 on MI355X (one machine): f16 NEOX 31.5 us per-thread, 28.4 us
// with no angles at all, 28.6 us pair-major with two batches in flight. f32,
// whose angles are shared by all 40 heads of a thread, is ~0.5 us faster
// per-thread (the two block barriers cost about what the reductions save).
// ELEM: element-wise loads and stores (rows that are only element-aligned).
// A: DenTable (angles evaluated in-kernel from the denominators) or TableArgs
// (angles read from tables; per-thread, no block barrier).
template <typename T, int P, bool INTERLEAVED, bool SPLIT, int U, bool PAIR_MAJOR, bool ELEM, typename A, bool FOLD>
__global__ __launch_bounds__(kThreads) void rope_kernel(T* q, int nq, T* k, int nk, const int32_t* __restrict__ pos,
                                                             int64_t ntok, int64_t seq, int head_dim, int half,
                                                             int lanes_per_tok, int toks_per_block,
                                                             int heads_per_group, float pos_scale, A den) {
    static_assert(INTERLEAVED || !SPLIT, "SPLIT is an interleaved layout");
    constexpr bool TAB = std::is_same<A, TableArgs>::value;
    static_assert(!(TAB && PAIR_MAJOR), "table angles are read per thread");
    static_assert(!(FOLD && PAIR_MAJOR), "pair-major angles are shared by a block's consecutive tokens");
    constexpr int R = (!INTERLEAVED || SPLIT) ? 2 : 1;
    constexpr int L = INTERLEAVED ? 2 * P : P;
    constexpr int NA = SPLIT ? 2 * P : P;
    // [pair][token] with a row stride of toks_per_block + 1 floats: the
    // pair-major writes and the token-major reads both spread over the banks.
    // toks_per_block · half <= kThreads · NA, so kThreads · NA + kMaxHalf covers it.
    constexpr int kAngles = kThreads * NA + kMaxHalf;
    __shared__ uint32_t inv_pio4[24];
    __shared__ int32_t pos_s[kThreads];
    __shared__ float cs_s[kAngles], sn_s[kAngles];
    const int tid = threadIdx.x;
    const int tib = tid / lanes_per_tok;
    const int lit = tid - tib * lanes_per_tok;
    const int64_t t_first = (int64_t)blockIdx.x * toks_per_block;
    // FOLD (launches of fewer tokens than a block holds): the block's token
    // slots take (token, head group) units, unit = group · ntok + token, so a
    // one-token step runs in one block instead of one block per head group.
    int64_t t;
    int h_begin;
    bool active;
    if constexpr (FOLD) {
        const int unit = blockIdx.x * toks_per_block + tib;
        const int grp = unit / (int)ntok;
        t = unit - grp * ntok;
        h_begin = grp * heads_per_group;
        active = tib < toks_per_block && h_begin < nq + nk;
    } else {
        t = t_first + tib;
        h_begin = blockIdx.y * heads_per_group;
        active = tib < toks_per_block && t < ntok;
    }
    const int i0 = lit * P;
    const int off[2] = {INTERLEAVED ? 2 * i0 : i0, INTERLEAVED ? 2 * i0 + half : i0 + half};
    // Pair of angle a (0 <= a < NA) of this thread.
    auto pair_of = [&](int a) { return SPLIT ? i0 + (a / P) * (half / 2) + a % P : i0 + a; };
    const int64_t b = active ? t / seq : 0;
    const int64_t s = active ? t - b * seq : 0;
    int h_end = h_begin + heads_per_group;
    if (h_end > nq + nk) h_end = nq + nk;

    // This lane's row in head 0 of q and of k; heads lie seq · head_dim
    // elements apart, so a head's row is the lane's base plus a block-uniform
    // offset (scalar arithmetic and one 64-bit add per head, instead of the
    // full per-lane index). The store recomputes it from the head index rather
    // than carrying the load's pointer across the loop: a carried pointer lost
    // its global address space and the half-type stores compiled to flat
    // stores (also counted by the LDS counter the angle reads wait on; the
    // loop-top wait for the next batch already drains every store, so the
    // time measured the same either way).
    const size_t hs = (size_t)seq * (size_t)head_dim;
    T* const qb = q + ((size_t)b * (size_t)nq * (size_t)seq + (size_t)s) * (size_t)head_dim;
    T* const kb = nk > 0 ? k + ((size_t)b * (size_t)nk * (size_t)seq + (size_t)s) * (size_t)head_dim : qb;
    auto row_of = [&](int hh) -> T* { return hh < nq ? qb + (size_t)hh * hs : kb + (size_t)(hh - nq) * hs; };
    auto load_batch = [&](int h0, RawRun<T, L, ELEM> (&buf)[U][R]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (h0 + u < h_end) {
                const T* row = row_of(h0 + u);
#pragma unroll
                for (int r = 0; r < R; ++r) buf[u][r].load(row + off[r]);
            }
        }
    };
    auto rotate_batch = [&](int h0, const RawRun<T, L, ELEM> (&buf)[U][R], const float (&cs)[NA],
                            const float (&sn)[NA]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (h0 + u < h_end) {
                T* row = row_of(h0 + u);
                if constexpr (!INTERLEAVED) {
                    float x0[P], x1[P], o0[P], o1[P];
                    buf[u][0].to_f32(x0);
                    buf[u][1].to_f32(x1);
#pragma unroll
                    for (int j = 0; j < P; ++j) {
                        o0[j] = x0[j] * cs[j] - x1[j] * sn[j];
                        o1[j] = x1[j] * cs[j] + x0[j] * sn[j];
                    }
                    store_run<T, P, ELEM>(row + off[0], o0);
                    store_run<T, P, ELEM>(row + off[1], o1);
                } else {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float x[2 * P], o[2 * P];
                        buf[u][r].to_f32(x);
#pragma unroll
                        for (int j = 0; j < P; ++j) {
                            o[2 * j] = x[2 * j] * cs[r * P + j] - x[2 * j + 1] * sn[r * P + j];
                            o[2 * j + 1] = x[2 * j + 1] * cs[r * P + j] + x[2 * j] * sn[r * P + j];
                        }
                        store_run<T, 2 * P, ELEM>(row + off[r], o);
                    }
                }
            }
        }
    };

    // The position load goes first: loads complete in order, so staging it
    // waits for it alone while the first two batches stay in flight.
    float cs[NA], sn[NA];
    constexpr int kPre = (PAIR_MAJOR && sizeof(T) == 2) ? 4 : 2;  // batches requested before the angles
    RawRun<T, L, ELEM> bufs[kPre][U][R];
    if constexpr (TAB) {
        // Token s's row of the tables: requested after the position (row pos[s])
        // and alongside the first two batches, so the thread waits on memory
        // for the position and then once more; no sin/cos, no block barrier.
        if (!active) return;
        const int32_t ps = pos != nullptr ? pos[s] : (int32_t)s;
        load_batch(h_begin, bufs[0]);
        load_batch(h_begin + U, bufs[1]);
        if (ps < 0 || (int64_t)ps >= den.rows) {
            if (den.bad != nullptr) *den.bad = 1;
            return;
        }
        const float* crow = den.cs + (size_t)ps * (size_t)half;
        const float* srow = den.sn + (size_t)ps * (size_t)half;
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            cs[a] = crow[pair_of(a)];
            sn[a] = srow[pair_of(a)];
        }
    } else if constexpr (PAIR_MAJOR) {
        int32_t pv = 0;
        if (tid < toks_per_block && t_first + tid < ntok) pv = pos[(t_first + tid) % seq];
        if (active) {
#pragma unroll
            for (int p = 0; p < kPre; ++p) load_batch(h_begin + p * U, bufs[p]);
        }
        if (tid < toks_per_block) pos_s[tid] = pv;
        if (tid < 24) inv_pio4[tid] = kInvPio4.w[tid];
        __syncthreads();

        const int stride = toks_per_block + 1;
        const int n_angles = toks_per_block * half;
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int a = j * kThreads + tid;
            if (a < n_angles) {
                const int pair = a / toks_per_block;
                const int tk = a - pair * toks_per_block;
                const float p = (float)pos_s[tk] / pos_scale;
                const float freq = p / den.v[pair];
                float sv, cv;
                glibc_sincosf_tab(freq, inv_pio4, &sv, &cv);
                cs_s[pair * stride + tk] = cv;
                sn_s[pair * stride + tk] = sv;
            }
        }
        __syncthreads();
        if (!active) return;
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            cs[a] = cs_s[pair_of(a) * stride + tib];
            sn[a] = sn_s[pair_of(a) * stride + tib];
        }
    } else {
        int32_t ps = 0;
        if (active) {
            ps = pos[s];
            load_batch(h_begin, bufs[0]);
            load_batch(h_begin + U, bufs[1]);
        }
        if (tid < 24) inv_pio4[tid] = kInvPio4.w[tid];
        __syncthreads();
        if (!active) return;
        const float p = (float)ps / pos_scale;
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            const float freq = p / den.v[pair_of(a)];
            glibc_sincosf_tab(freq, inv_pio4, &sn[a], &cs[a]);
        }
    }

    // The batches requested before the angles, in order; the first two are
    // refilled with the next two batches (load_batch and rotate_batch skip
    // heads past the group's end).
    int h_loop = h_begin;
    if constexpr (kPre > 2) {
#pragma unroll
        for (int p = 0; p < kPre; ++p) {
            rotate_batch(h_begin + p * U, bufs[p], cs, sn);
            if (p < 2) load_batch(h_begin + (kPre + p) * U, bufs[p]);
        }
        h_loop = h_begin + kPre * U;
    }
    // Two batches alternate: while one is rotated and stored, the other's
    // loads are in flight.
    for (int h0 = h_loop; h0 < h_end; h0 += 2 * U) {
        rotate_batch(h0, bufs[0], cs, sn);
        if (h0 + 2 * U < h_end) load_batch(h0 + 2 * U, bufs[0]);
        if (h0 + U >= h_end) break;
        rotate_batch(h0 + U, bufs[1], cs, sn);
        if (h0 + 3 * U < h_end) load_batch(h0 + 3 * U, bufs[1]);
    }
}

// Fused decode step: heads [0, nq) are q rows, rotated and written to qo
// heads-major; heads [nq, nq + nkv) rotate the k row and write it, plus the v
// row, to cache row (h, positions[s]). batch = 1 and rotary_dim = head_dim, so
// a thread's P pairs and the pairs of its lane neighbours cover every channel
// of the row. TM: q, k and v are read token-major [seq, heads, head_dim] (the
// projections' layout) instead of heads-major; without TM, qo == q (in place).
template <typename T, typename TC, typename TB, int P, bool INTERLEAVED, bool TM>
__global__ __launch_bounds__(kThreads) void rope_kv_kernel(const T* q, T* qo, int nq, const T* __restrict__ k,
                                                           const T* __restrict__ v, int nkv,
                                                           const int32_t* __restrict__ pos, int64_t seq, int head_dim,
                                                           int half, int lanes_per_tok, int toks_per_block,
                                                           int heads_per_group, float pos_scale, TC* kc, TC* vc,
                                                           int64_t max_seq, int32_t* bad_pos_flag, const TB* bq,
                                                           const TB* bk, const TB* bv, DenTable den,
                                                           const float* __restrict__ ang, bool ang_by_pos) {
    __shared__ uint32_t inv_pio4[24];
    const int tib = threadIdx.x / lanes_per_tok;
    const int lit = threadIdx.x - tib * lanes_per_tok;
    const int64_t s = (int64_t)blockIdx.x * toks_per_block + tib;
    const bool active = tib < toks_per_block && s < seq;
    const int i0 = lit * P;
    // Element offsets of this thread's two runs of P elements within a row.
    const int a0 = INTERLEAVED ? 2 * i0 : i0;
    const int a1 = INTERLEAVED ? 2 * i0 + P : i0 + half;
    const int h_begin = blockIdx.y * heads_per_group;
    int h_end = h_begin + heads_per_group;
    if (h_end > nq + nkv) h_end = nq + nkv;

    // Row (head h, token s) of a [heads, seq, hd] (or, TM, [seq, heads, hd]) tensor.
    auto row_of = [&](const T* base, int heads, int h) {
        return base + (TM ? (size_t)s * (size_t)heads + (size_t)h : (size_t)h * (size_t)seq + (size_t)s) *
                          (size_t)head_dim;
    };
    // Row values with the bias of their channels added (y + b in f32, then
    // stored in the activation type before RoPE reads it: round through T).
    auto load_row = [&](const T* row, const TB* bias, float (&u0)[P], float (&u1)[P]) {
        if constexpr (!INTERLEAVED) {
            load_f32<T, P, true>(row + a0, u0);
            load_f32<T, P, true>(row + a1, u1);
        } else {
            float x[2 * P];
            load_f32<T, 2 * P, true>(row + a0, x);
#pragma unroll
            for (int j = 0; j < P; ++j) {
                u0[j] = x[2 * j];
                u1[j] = x[2 * j + 1];
            }
        }
        if (bias != nullptr) {
            float b0[P], b1[P];
            if constexpr (!INTERLEAVED) {
                load_f32<TB, P>(bias + a0, b0);
                load_f32<TB, P>(bias + a1, b1);
            } else {
                float b[2 * P];
                load_f32<TB, 2 * P>(bias + a0, b);
#pragma unroll
                for (int j = 0; j < P; ++j) {
                    b0[j] = b[2 * j];
                    b1[j] = b[2 * j + 1];
                }
            }
#pragma unroll
            for (int j = 0; j < P; ++j) {
                u0[j] = widen(narrow<T>(u0[j] + b0[j]));
                u1[j] = widen(narrow<T>(u1[j] + b1[j]));
            }
        }
    };

    // The position and the first head's rows need neither the angle nor the
    // table: they are issued before the table is staged, so the block waits
    // on memory once instead of three times (what a one-token decode step
    // costs is mostly these latencies).
    int32_t ps = 0;
    float x0[P], x1[P], v0[P], v1[P];
    // A head's input rows: q (heads < nq), or k and v. (A macro: a lambda taking
    // these arrays by reference left them in scratch memory for P = 1.)
#define SPH_LOAD_HEAD(hh)                                                                         \
    do {                                                                                          \
        if ((hh) < nq) {                                                                          \
            load_row(row_of(q, nq, (hh)), bq ? bq + (size_t)(hh) * head_dim : nullptr, x0, x1);   \
        } else {                                                                                  \
            const int h_ = (hh) - nq;                                                             \
            load_row(row_of(k, nkv, h_), bk ? bk + (size_t)h_ * head_dim : nullptr, x0, x1);      \
            load_row(row_of(v, nkv, h_), bv ? bv + (size_t)h_ * head_dim : nullptr, v0, v1);      \
        }                                                                                         \
    } while (0)
    float cs[P], sn[P];
    if (ang != nullptr && !ang_by_pos) {
        // Angles supplied per (token, pair) as (cos, sin): requested with the
        // position and the rows, so the step waits on memory once and computes
        // no sin/cos (the whole block takes this branch; no barrier follows).
        if (!active) return;
        ps = pos[s];
        const float* a = ang + 2 * ((size_t)s * (size_t)half + (size_t)i0);
#pragma unroll
        for (int j = 0; j < P; ++j) {
            cs[j] = a[2 * j];
            sn[j] = a[2 * j + 1];
        }
        if (h_begin < h_end) SPH_LOAD_HEAD(h_begin);
    } else if (ang != nullptr) {
        // Angles read from row pos[s] of a per-position table of max_seq rows
        // (the first head's rows are requested before the position is waited
        // on). A position outside [0, max_seq) reads no row: q is rotated by
        // angle 0 (cos 1, sin 0), the caches are left alone and the flag set.
        if (!active) return;
        ps = pos[s];
        if (h_begin < h_end) SPH_LOAD_HEAD(h_begin);
        const bool in_table = ps >= 0 && (int64_t)ps < max_seq;
        const float* a = ang + 2 * ((size_t)(in_table ? ps : 0) * (size_t)half + (size_t)i0);
#pragma unroll
        for (int j = 0; j < P; ++j) {
            cs[j] = in_table ? a[2 * j] : 1.0f;
            sn[j] = in_table ? a[2 * j + 1] : 0.0f;
        }
    } else {
        if (active) {
            ps = pos[s];
            if (h_begin < h_end) SPH_LOAD_HEAD(h_begin);
        }
        const uint32_t* tab = stage_inv_pio4(inv_pio4);
        if (!active) return;
        const float p = (float)ps / pos_scale;
#pragma unroll
        for (int j = 0; j < P; ++j) {
            const float freq = p / den.v[i0 + j];
            glibc_sincosf_tab(freq, tab, &sn[j], &cs[j]);
        }
    }
    const bool pos_ok = ps >= 0 && (int64_t)ps < max_seq;
    if (!pos_ok && bad_pos_flag != nullptr && lit == 0 && blockIdx.y == 0) *bad_pos_flag = 1;

    auto put = [&](auto* row, const float (&u0)[P], const float (&u1)[P]) {
        using TR = typename std::remove_pointer<decltype(row)>::type;
        if constexpr (!INTERLEAVED) {
            store_f32<TR, P, true>(row + a0, u0);
            store_f32<TR, P, true>(row + a1, u1);
        } else {
            float o[2 * P];
#pragma unroll
            for (int j = 0; j < P; ++j) {
                o[2 * j] = u0[j];
                o[2 * j + 1] = u1[j];
            }
            store_f32<TR, 2 * P, true>(row + a0, o);
        }
    };
    for (int hh = h_begin; hh < h_end; ++hh) {
        const bool is_q = hh < nq;
        if (hh != h_begin) SPH_LOAD_HEAD(hh);
        if (!is_q && !pos_ok) continue;
        float o0[P], o1[P];
#pragma unroll
        for (int j = 0; j < P; ++j) {
            o0[j] = x0[j] * cs[j] - x1[j] * sn[j];
            o1[j] = x1[j] * cs[j] + x0[j] * sn[j];
        }
        if (is_q) {
            put(qo + ((size_t)hh * (size_t)seq + (size_t)s) * (size_t)head_dim, o0, o1);
        } else {
            const size_t crow = ((size_t)(hh - nq) * (size_t)max_seq + (size_t)ps) * (size_t)head_dim;
            // The unfused sequence stores rotated k in the activation type
            // before converting it to the cache type: round through T first.
            if constexpr (!std::is_same<T, float>::value) {
#pragma unroll
                for (int j = 0; j < P; ++j) {
                    o0[j] = widen(narrow<T>(o0[j]));
                    o1[j] = widen(narrow<T>(o1[j]));
                }
            }
            put(kc + crow, o0, o1);
            put(vc + crow, v0, v1);  // v: the same channels, moved unrotated
        }
    }
#undef SPH_LOAD_HEAD
}

// Launch shape of rope_kernel per storage type and layout, chosen by
// round-robin timing at the Llama-3-8B shape on MI355X (32 + 8 heads × 8192
// tokens × 128, in place), beside an in-place 16-byte copy of the same bytes
// (two launches, q and k) as the ceiling; medians of 12 rounds on one machine:
//  - half types: NEOX P = 4 (8-byte runs), interleaved split with P = 2
//    (two 8-byte runs), U = 2, pair-major angles, 2048 units in all (four
//    head groups, each recomputing its angles: more waves in flight outweigh
//    the repeated angle work). f16 NEOX 31.0 µs, interleaved 30.6 µs, copy
//    30.2 µs with two batches requested before the angles; four: 28.4 µs
//    both. U = 4 cost 2–3 µs, P = 8 or one run of P = 4 0.3–4 µs.
//  - f32: P = 4 NEOX, interleaved split with P = 2 (16-byte runs), U = 1,
//    per-thread angles, 512 units (one group holds all 40 heads). NEOX
//    57.5 µs, interleaved 58.0 µs (one 16-byte run: 61.2 µs), copy 56.3 µs.
// Machines differ by up to ±5 % in absolute speed; the ordering held on each.
template <typename T, bool IL>
struct RopeShape {
    static constexpr bool kHalf = sizeof(T) == 2;
    static constexpr int P = IL ? 2 : 4;  // preferred pairs per run
    static constexpr bool kSplit = IL;
    static constexpr int U = kHalf ? 2 : 1;
    static constexpr bool kPairMajor = kHalf;
    static constexpr int kTarget = kHalf ? 2048 : 512;
};

// target: blocks to aim for in all (token blocks × head groups).
// Table angles are read per thread, so those launches never take the pair-major shape.
template <typename T, int P, bool IL, bool SPLIT = RopeShape<T, IL>::kSplit, int U = RopeShape<T, IL>::U,
          bool PM = RopeShape<T, IL>::kPairMajor, bool ELEM = false, typename A = DenTable>
int launch_rope_p(T* q, int nq, T* k, int nk, const int32_t* pos, int64_t ntok, int64_t seq, int head_dim,
                  int half, float pos_scale, const A& den, hipStream_t stream,
                  int target = RopeShape<T, IL>::kTarget) {
    constexpr bool kPM = PM && !std::is_same<A, TableArgs>::value;
    const int lanes_per_tok = half / (SPLIT ? 2 * P : P);
    const int toks_per_block = kThreads / lanes_per_tok;
    const int64_t blocks_x = (ntok + toks_per_block - 1) / toks_per_block;
    const int heads = nq + nk;
    int groups = (int)((target + blocks_x - 1) / blocks_x);
    if (groups > heads) groups = heads;
    if (groups < 1) groups = 1;
    const int heads_per_group = (heads + groups - 1) / groups;
    groups = (heads + heads_per_group - 1) / heads_per_group;
    if (blocks_x > INT32_MAX) return SPH_EINVAL;
    if constexpr (!kPM) {
        // Fewer tokens than a block holds: (token, head group) units share blocks (FOLD).
        if (ntok < toks_per_block) {
            const int64_t units = ntok * (int64_t)groups;  // < toks_per_block · heads
            const dim3 grid((unsigned)((units + toks_per_block - 1) / toks_per_block));
            return launch(rope_kernel<T, P, IL, SPLIT, U, false, ELEM, A, true>, grid, kThreads, stream, q, nq, k, nk,
                          pos, ntok, seq, head_dim, half, lanes_per_tok, toks_per_block, heads_per_group, pos_scale,
                          den);
        }
    }
    const dim3 grid((unsigned)blocks_x, (unsigned)groups);
    return launch(rope_kernel<T, P, IL, SPLIT, U, kPM, ELEM, A, false>, grid, kThreads, stream, q, nq, k, nk, pos,
                  ntok, seq, head_dim, half, lanes_per_tok, toks_per_block, heads_per_group, pos_scale, den);
}

// Denominators powf(base, 2i / rotary_dim) from the host libm, the call the reference makes.
inline void fill_dens(DenTable& den, int half, int rotary_dim, float base) {
    for (int i = 0; i < kMaxHalf; ++i)
        den.v[i] = i < half ? powf(base, 2.0f * (float)i / (float)rotary_dim) : 1.0f;
}

template <typename T, typename TC, typename TB, int P, bool IL, bool TM>
int launch_rope_kv_p(const T* q, T* qo, int nq, const T* k, const T* v, int nkv, const int32_t* pos, int64_t seq, int head_dim,
                     float pos_scale, TC* kc, TC* vc, int64_t max_seq, int32_t* flag, const TB* bq, const TB* bk,
                     const TB* bv, const DenTable& den, const float* ang, bool ang_by_pos, hipStream_t stream) {
    const int half = head_dim / 2;
    const int lanes_per_tok = half / P;
    const int toks_per_block = kThreads / lanes_per_tok;
    const int64_t blocks_x = (seq + toks_per_block - 1) / toks_per_block;
    const int heads = nq + nkv;
    // Blocks to aim for (head groups × token blocks), swept at the Llama-3-8B
    // shape: f32 512; half types 512 NEOX, 1536 interleaved.
    const int target = sizeof(T) == 4 ? 512 : (IL ? 1536 : 512);
    int groups = (int)((target + blocks_x - 1) / blocks_x);
    if (groups > heads) groups = heads;
    if (groups < 1) groups = 1;
    const int heads_per_group = (heads + groups - 1) / groups;
    groups = (heads + heads_per_group - 1) / heads_per_group;
    if (blocks_x > INT32_MAX) return SPH_EINVAL;
    const dim3 grid((unsigned)blocks_x, (unsigned)groups);
    return launch(rope_kv_kernel<T, TC, TB, P, IL, TM>, grid, kThreads, stream, q, qo, nq, k, v, nkv, pos, seq,
                  head_dim, half, lanes_per_tok, toks_per_block, heads_per_group, pos_scale, kc, vc, max_seq, flag, bq,
                  bk, bv, den, ang, ang_by_pos);
}

// P: pairs per thread, the widest whose accesses of q/k/v (type T) and of the
// caches (type TC) stay within 16 bytes and aligned.
template <typename T, typename TC, typename TB, bool TM>
int launch_rope_kv(const void* qv, void* qov, int nq, const void* kv, const void* vv, int nkv, int layout,
                   const int32_t* pos, int64_t seq, int head_dim, float base, float pos_scale, void* kcv, void* vcv,
                   int64_t max_seq, int32_t* flag, const void* bqv, const void* bkv, const void* bvv, const float* ang,
                   bool ang_by_pos, hipStream_t stream) {
    const TB* bq = static_cast<const TB*>(bqv);
    const TB* bk = static_cast<const TB*>(bkv);
    const TB* bv = static_cast<const TB*>(bvv);
    const T* q = static_cast<const T*>(qv);
    T* qo = static_cast<T*>(qov);
    const T* k = static_cast<const T*>(kv);
    const T* v = static_cast<const T*>(vv);
    TC* kc = static_cast<TC*>(kcv);
    TC* vc = static_cast<TC*>(vcv);
    const int half = head_dim / 2;
    // Supplied angles leave the denominators unused: no libm calls per launch.
    DenTable den{};
    if (ang == nullptr) fill_dens(den, half, head_dim, base);
    const bool il = layout == SPH_ROPE_INTERLEAVED;
    auto ok = [&](int P) {
        const int run = il ? 2 * P : P;  // contiguous elements per access
        if (half % P != 0 || head_dim % run != 0) return false;
        if (run * sizeof(T) > 16 || run * sizeof(TC) > 16) return false;
        if ((run * sizeof(T)) % 4 != 0 || (run * sizeof(TC)) % 4 != 0) return false;
        const size_t at = run * sizeof(T) < 16 ? run * sizeof(T) : 16;
        const size_t ac = run * sizeof(TC) < 16 ? run * sizeof(TC) : 16;
        const size_t ab = run * sizeof(TB) < 16 ? run * sizeof(TB) : 16;  // bias runs may span two 16-byte loads
        return aligned(q, at) && aligned(qo, at) && aligned(k, at) && aligned(v, at) && aligned(kc, ac) &&
               aligned(vc, ac) && aligned(bq, ab) && aligned(bk, ab) && aligned(bv, ab);
    };
    constexpr int V = vec16<T>::n < vec16<TC>::n ? vec16<T>::n : vec16<TC>::n;
    // A decode step (a few tokens) leaves most lanes of its blocks idle and its
    // time is one dependent chain — position load, the thread's sin/cos, store —
    // so it takes the narrowest runs that stay word-sized: fewer angles per lane.
    const bool few = seq <= 4;
    if (!il) {
        if (few && ok(V / 2)) return launch_rope_kv_p<T, TC, TB, V / 2, false, TM>(q, qo, nq, k, v, nkv, pos, seq, head_dim, pos_scale, kc, vc, max_seq, flag, bq, bk, bv, den, ang, ang_by_pos, stream);
        if (ok(V)) return launch_rope_kv_p<T, TC, TB, V, false, TM>(q, qo, nq, k, v, nkv, pos, seq, head_dim, pos_scale, kc, vc, max_seq, flag, bq, bk, bv, den, ang, ang_by_pos, stream);
        if (ok(V / 2)) return launch_rope_kv_p<T, TC, TB, V / 2, false, TM>(q, qo, nq, k, v, nkv, pos, seq, head_dim, pos_scale, kc, vc, max_seq, flag, bq, bk, bv, den, ang, ang_by_pos, stream);
        if constexpr (V / 4 >= 2) {
            if (ok(V / 4)) return launch_rope_kv_p<T, TC, TB, V / 4, false, TM>(q, qo, nq, k, v, nkv, pos, seq, head_dim, pos_scale, kc, vc, max_seq, flag, bq, bk, bv, den, ang, ang_by_pos, stream);
        }
    } else {
        if constexpr (V / 4 >= 1) {
            if (few && ok(V / 4)) return launch_rope_kv_p<T, TC, TB, V / 4, true, TM>(q, qo, nq, k, v, nkv, pos, seq, head_dim, pos_scale, kc, vc, max_seq, flag, bq, bk, bv, den, ang, ang_by_pos, stream);
        }
        if (ok(V / 2)) return launch_rope_kv_p<T, TC, TB, V / 2, true, TM>(q, qo, nq, k, v, nkv, pos, seq, head_dim, pos_scale, kc, vc, max_seq, flag, bq, bk, bv, den, ang, ang_by_pos, stream);
        if constexpr (V / 4 >= 1) {
            if (ok(V / 4)) return launch_rope_kv_p<T, TC, TB, V / 4, true, TM>(q, qo, nq, k, v, nkv, pos, seq, head_dim, pos_scale, kc, vc, max_seq, flag, bq, bk, bv, den, ang, ang_by_pos, stream);
        }
    }
    return SPH_EINVAL;  // head_dim or alignment the vector paths do not cover
}

constexpr int64_t kFewRopeRows = int64_t(1) << 15;

// den: the denominators (DenTable) or the angle tables (TableArgs).
template <typename T, typename A>
int launch_rope(void* qv, int nq, void* kv, int nk, int layout, const int32_t* pos, int64_t batch, int64_t seq,
                int head_dim, int rotary_dim, float pos_scale, const A& den, hipStream_t stream) {
    T* q = static_cast<T*>(qv);
    T* k = static_cast<T*>(kv);
    const int half = rotary_dim / 2;
    const int64_t ntok = batch * seq;
    auto ok = [&](int P, int elems_per_access) {
        const size_t bytes = (size_t)elems_per_access * sizeof(T);
        if (half % P != 0 || head_dim % elems_per_access != 0) return false;
        if (elems_per_access > 1 && bytes % 4 != 0) return false;
        return aligned(q, bytes < 16 ? bytes : 16) && (k == nullptr || aligned(k, bytes < 16 ? bytes : 16));
    };
    if (layout == SPH_ROPE_NEOX) {
        // The preferred P (a run of P elements per access), then narrower runs.
        constexpr int PN = RopeShape<T, false>::P;
        // In-kernel angles at up to 2^15 (token, head) rows (a decode step, a small prefill chunk):
        // one pair per run, so each lane evaluates one sin/cos — the long pole of a small launch.
        // Per launch, back to back on MI355X, Qwen2.5-0.5B's 14 + 2 heads x 64: T = 1 f32 3.0 -> 2.25
        // µs, f16 4.0 -> 2.57; T = 512 f32 3.96 -> 3.03, f16 4.37 -> 3.61; T = 2048 f32 5.0 -> 4.7,
        // f16 6.3 -> 5.9. Table angles gain nothing from it (T = 512 f32 2.44 -> 2.66).
        if constexpr (std::is_same<A, DenTable>::value) {
            if (ntok * (int64_t)(nq + nk) <= kFewRopeRows && ok(1, 1))
                return launch_rope_p<T, 1, false>(q, nq, k, nk, pos, ntok, seq, head_dim, half, pos_scale, den, stream);
        }
        if (ok(PN, PN)) return launch_rope_p<T, PN, false>(q, nq, k, nk, pos, ntok, seq, head_dim, half, pos_scale, den, stream);
        if constexpr (PN / 2 >= 2) {
            if (ok(PN / 2, PN / 2)) return launch_rope_p<T, PN / 2, false>(q, nq, k, nk, pos, ntok, seq, head_dim, half, pos_scale, den, stream);
        }
        if constexpr (PN / 4 >= 2) {
            if (ok(PN / 4, PN / 4)) return launch_rope_p<T, PN / 4, false>(q, nq, k, nk, pos, ntok, seq, head_dim, half, pos_scale, den, stream);
        }
        return launch_rope_p<T, 1, false>(q, nq, k, nk, pos, ntok, seq, head_dim, half, pos_scale, den, stream);
    }

    // Interleaved: split runs (two per thread, from both halves of the pairs)
    // when half divides into them, else one run per thread.
    constexpr int PI = RopeShape<T, true>::P;
    // In-kernel angles at small launches: one pair per run, as for NEOX (T = 1 f32 3.05 -> 2.24 µs,
    // f16 4.0 -> 2.5; T = 512 f32 3.85 -> 3.02, f16 4.37 -> 3.65; T = 2048 f16 6.33 -> 5.71).
    if constexpr (std::is_same<A, DenTable>::value) {
        if (ntok * (int64_t)(nq + nk) <= kFewRopeRows && ok(1, 2))
            return launch_rope_p<T, 1, true, false>(q, nq, k, nk, pos, ntok, seq, head_dim, half, pos_scale, den, stream);
    }
    if (half % (2 * PI) == 0 && ok(PI, 2 * PI))
        return launch_rope_p<T, PI, true, true>(q, nq, k, nk, pos, ntok, seq, head_dim, half, pos_scale, den, stream);
    constexpr int V = vec16<T>::n;  // elements per 16-byte access
    if (ok(V / 2, V)) return launch_rope_p<T, V / 2, true, false>(q, nq, k, nk, pos, ntok, seq, head_dim, half, pos_scale, den, stream);
    if constexpr (V / 4 >= 1) {
        if (ok(V / 4, V / 2)) return launch_rope_p<T, V / 4, true, false>(q, nq, k, nk, pos, ntok, seq, head_dim, half, pos_scale, den, stream);
    }
    // Rows only element-aligned: element accesses (a 2-element run would not be word-aligned).
    return launch_rope_p<T, 1, true, false, RopeShape<T, true>::U, RopeShape<T, true>::kPairMajor, true>(
        q, nq, k, nk, pos, ntok, seq, head_dim, half, pos_scale, den, stream);
}

}  // namespace
}  // namespace sph

extern "C" int sph_rope(void* q, int64_t n_q_heads, void* k, int64_t n_k_heads, int dtype, int layout,
                        const int32_t* positions, int64_t batch, int64_t seq, int64_t head_dim,
                        int64_t rotary_dim, float base, float pos_scale, void* stream) {
    if (layout != SPH_ROPE_NEOX && layout != SPH_ROPE_INTERLEAVED) return SPH_EINVAL;
    if (!sph::is_float_dtype(dtype)) return SPH_EINVAL;
    if (k == nullptr) n_k_heads = 0;
    if (n_q_heads < 0 || n_k_heads < 0 || batch < 0 || seq < 0) return SPH_EINVAL;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > INT32_MAX) return SPH_EINVAL;
    if (rotary_dim <= 0 || rotary_dim % 2 != 0 || rotary_dim > head_dim || rotary_dim / 2 > sph::kMaxHalf)
        return SPH_EINVAL;
    if (n_q_heads + n_k_heads > INT32_MAX) return SPH_EINVAL;
    const int64_t heads = n_q_heads + n_k_heads;
    if (batch == 0 || seq == 0 || heads == 0) return SPH_OK;
    if (positions == nullptr || (n_q_heads > 0 && q == nullptr)) return SPH_EINVAL;
    if (!(pos_scale == pos_scale) || pos_scale == 0.0f) return SPH_EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // The reference's denominators: base.powf(2.0 * i as f32 / rotary_dim as f32), host libm.
    sph::DenTable den;
    sph::fill_dens(den, (int)rotary_dim / 2, (int)rotary_dim, base);
    return sph::with_float_type(dtype, [&](auto t) -> int {
        using T = decltype(t);
        return sph::launch_rope<T>(q, (int)n_q_heads, k, (int)n_k_heads, layout, positions, batch, seq, (int)head_dim,
                                   (int)rotary_dim, pos_scale, den, s);
    });
}

extern "C" int sph_rope_cached(void* q, int64_t n_q_heads, void* k, int64_t n_k_heads, int dtype, int layout,
                               const float* cos_table, const float* sin_table, int64_t table_rows,
                               const int32_t* positions, int64_t batch, int64_t seq, int64_t head_dim,
                               int64_t rotary_dim, int32_t* bad_pos_flag, void* stream) {
    if (layout != SPH_ROPE_NEOX && layout != SPH_ROPE_INTERLEAVED) return SPH_EINVAL;
    if (!sph::is_float_dtype(dtype)) return SPH_EINVAL;
    if (k == nullptr) n_k_heads = 0;
    if (n_q_heads < 0 || n_k_heads < 0 || batch < 0 || seq < 0 || table_rows < 0) return SPH_EINVAL;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > INT32_MAX) return SPH_EINVAL;
    if (rotary_dim <= 0 || rotary_dim % 2 != 0 || rotary_dim > head_dim || rotary_dim / 2 > sph::kMaxHalf)
        return SPH_EINVAL;
    if (n_q_heads + n_k_heads > INT32_MAX) return SPH_EINVAL;
    const int64_t heads = n_q_heads + n_k_heads;
    if (batch == 0 || seq == 0 || heads == 0) return SPH_OK;
    if (n_q_heads > 0 && q == nullptr) return SPH_EINVAL;
    if (cos_table == nullptr || sin_table == nullptr || !sph::aligned(cos_table, 4) || !sph::aligned(sin_table, 4))
        return SPH_EINVAL;
    // Without positions token s reads row s: the tables must hold seq rows.
    if (positions == nullptr && table_rows < seq) return SPH_ERANGE;
    if (seq > INT32_MAX) return SPH_EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const sph::TableArgs tab{cos_table, sin_table, table_rows, bad_pos_flag};
    return sph::with_float_type(dtype, [&](auto t) -> int {
        using T = decltype(t);
        return sph::launch_rope<T>(q, (int)n_q_heads, k, (int)n_k_heads, layout, positions, batch, seq, (int)head_dim,
                                   (int)rotary_dim, 1.0f, tab, s);
    });
}

// Host-side table builder: the reference's angle, (pos as f32 / pos_scale) /
// base.powf(2i / rotary_dim) (rope.rs:48-50, :123-125), and its sin / cos, with
// the host libm the reference's f32::sin_cos / powf bind to.
extern "C" int sph_rope_table(const int64_t* positions, int64_t n, int64_t rotary_dim, float base, float pos_scale,
                              float* cos_out, float* sin_out) {
    if (n < 0 || rotary_dim <= 0 || rotary_dim % 2 != 0) return SPH_EINVAL;
    if (!(pos_scale == pos_scale) || pos_scale == 0.0f) return SPH_EINVAL;
    if (n == 0) return SPH_OK;
    if (cos_out == nullptr || sin_out == nullptr) return SPH_EINVAL;
    const int64_t half = rotary_dim / 2;
    if (positions != nullptr)
        for (int64_t r = 0; r < n; ++r)
            if (positions[r] < 0) return SPH_EINVAL;
    float den[sph::kMaxHalf];
    const bool small = half <= sph::kMaxHalf;
    if (small)
        for (int64_t i = 0; i < half; ++i) den[i] = powf(base, 2.0f * (float)i / (float)rotary_dim);
    for (int64_t r = 0; r < n; ++r) {
        const int64_t pos = positions != nullptr ? positions[r] : r;
        const float p = (float)pos / pos_scale;
        for (int64_t i = 0; i < half; ++i) {
            const float d = small ? den[i] : powf(base, 2.0f * (float)i / (float)rotary_dim);
            const float freq = p / d;
            cos_out[r * half + i] = cosf(freq);
            sin_out[r * half + i] = sinf(freq);
        }
    }
    return SPH_OK;
}

namespace sph {
namespace {

// Validation and dispatch shared by the two fused entry points.
template <bool TM>
int rope_kv_entry(const void* q, void* q_out, int64_t n_q_heads, const void* k, const void* v, int64_t n_kv_heads,
                  int dtype, int layout, const int32_t* positions, int64_t seq, int64_t head_dim, float base,
                  float pos_scale, void* kcache, void* vcache, int cache_dtype, int64_t max_seq, const void* bq,
                  const void* bk, const void* bv, int bias_dtype, int32_t* bad_pos_flag, void* stream,
                  const float* angles = nullptr, bool angles_by_position = false) {
    if (layout != SPH_ROPE_NEOX && layout != SPH_ROPE_INTERLEAVED) return SPH_EINVAL;
    if (!is_float_dtype(dtype) || !is_float_dtype(cache_dtype)) return SPH_EINVAL;
    if ((bq || bk || bv) && !is_float_dtype(bias_dtype)) return SPH_EINVAL;
    if (!(bq || bk || bv)) bias_dtype = SPH_F32;
    if (n_q_heads < 0 || n_kv_heads < 0 || seq < 0 || max_seq < 0) return SPH_EINVAL;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim / 2 > kMaxHalf) return SPH_EINVAL;
    if (n_q_heads + n_kv_heads > INT32_MAX) return SPH_EINVAL;
    if (seq == 0 || n_q_heads + n_kv_heads == 0) return SPH_OK;
    if (positions == nullptr || (n_q_heads > 0 && (q == nullptr || q_out == nullptr))) return SPH_EINVAL;
    if (n_kv_heads > 0 && (k == nullptr || v == nullptr || kcache == nullptr || vcache == nullptr)) return SPH_EINVAL;
    if (!(pos_scale == pos_scale) || pos_scale == 0.0f) return SPH_EINVAL;
    if (TM && n_q_heads > 0) {  // q_out is written while q is still being read: they must not overlap
        const uintptr_t bytes = (uintptr_t)n_q_heads * (uintptr_t)seq * (uintptr_t)head_dim * dtype_size(dtype);
        const uintptr_t a = (uintptr_t)q, b = (uintptr_t)q_out;
        if (a < b + bytes && b < a + bytes) return SPH_EINVAL;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    return with_float_type(dtype, [&](auto t) -> int {
        using T = decltype(t);
        return with_float_type(cache_dtype, [&](auto tc) -> int {
            using TC = decltype(tc);
            return with_float_type(bias_dtype, [&](auto tb) -> int {
                using TB = decltype(tb);
                return launch_rope_kv<T, TC, TB, TM>(q, q_out, (int)n_q_heads, k, v, (int)n_kv_heads, layout,
                                                     positions, seq, (int)head_dim, base, pos_scale, kcache, vcache,
                                                     max_seq, bad_pos_flag, bq, bk, bv, angles,
                                                     angles_by_position, s);
            });
        });
    });
}

}  // namespace
}  // namespace sph

extern "C" int sph_rope_kv_append(void* q, int64_t n_q_heads, const void* k, const void* v, int64_t n_kv_heads,
                                  int dtype, int layout, const int32_t* positions, int64_t seq, int64_t head_dim,
                                  float base, float pos_scale, void* kcache, void* vcache, int cache_dtype,
                                  int64_t max_seq, const void* bq, const void* bk, const void* bv, int bias_dtype,
                                  int32_t* bad_pos_flag, void* stream) {
    return sph::rope_kv_entry<false>(q, q, n_q_heads, k, v, n_kv_heads, dtype, layout, positions, seq, head_dim, base,
                                     pos_scale, kcache, vcache, cache_dtype, max_seq, bq, bk, bv, bias_dtype,
                                     bad_pos_flag, stream);
}

// Declared in sph_internal.h (not exported).
extern "C" int sph_rope_kv_append_angles(void* q, int64_t n_q_heads, const void* k, const void* v, int64_t n_kv_heads,
                                         int dtype, int layout, const int32_t* positions, const float* angles,
                                         int64_t seq, int64_t head_dim, void* kcache, void* vcache, int cache_dtype,
                                         int64_t max_seq, const void* bq, const void* bk, const void* bv,
                                         int bias_dtype, int32_t* bad_pos_flag, void* stream) {
    if (angles == nullptr || !sph::aligned(angles, 8)) return SPH_EINVAL;
    return sph::rope_kv_entry<false>(q, q, n_q_heads, k, v, n_kv_heads, dtype, layout, positions, seq, head_dim, 1.0f,
                                     1.0f, kcache, vcache, cache_dtype, max_seq, bq, bk, bv, bias_dtype, bad_pos_flag,
                                     stream, angles);
}

extern "C" int sph_rope_kv_append_tokens(const void* q, void* q_out, int64_t n_q_heads, const void* k, const void* v,
                                         int64_t n_kv_heads, int dtype, int layout, const int32_t* positions,
                                         int64_t seq, int64_t head_dim, float base, float pos_scale, void* kcache,
                                         void* vcache, int cache_dtype, int64_t max_seq, const void* bq,
                                         const void* bk, const void* bv, int bias_dtype, int32_t* bad_pos_flag,
                                         void* stream) {
    return sph::rope_kv_entry<true>(q, q_out, n_q_heads, k, v, n_kv_heads, dtype, layout, positions, seq, head_dim,
                                    base, pos_scale, kcache, vcache, cache_dtype, max_seq, bq, bk, bv, bias_dtype,
                                    bad_pos_flag, stream);
}

// Declared in sph_internal.h (not exported).
extern "C" int sph_rope_kv_append_tokens_angles(const void* q, void* q_out, int64_t n_q_heads, const void* k,
                                                const void* v, int64_t n_kv_heads, int dtype, int layout,
                                                const int32_t* positions, const float* angles, int64_t seq,
                                                int64_t head_dim, void* kcache, void* vcache, int cache_dtype,
                                                int64_t max_seq, const void* bq, const void* bk, const void* bv,
                                                int bias_dtype, int32_t* bad_pos_flag, void* stream) {
    if (angles == nullptr || !sph::aligned(angles, 8)) return SPH_EINVAL;
    return sph::rope_kv_entry<true>(q, q_out, n_q_heads, k, v, n_kv_heads, dtype, layout, positions, seq, head_dim,
                                    1.0f, 1.0f, kcache, vcache, cache_dtype, max_seq, bq, bk, bv, bias_dtype,
                                    bad_pos_flag, stream, angles, true);
}
