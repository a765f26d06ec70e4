/*
 * sapient_hip.h — C ABI of the MI355X (gfx950) fused per-layer op set.
 *
 * This is the drop-in boundary: a Rust backend crate (or any FFI caller)
 * binds these symbols and wraps them behind sapient's op traits. Every
 * function:
 *   - takes raw DEVICE pointers, explicit sizes and a HIP stream
 *     (`stream` is a hipStream_t passed as void*; NULL = the default stream);
 *     a device pointer is any address the kernels can reach: device memory,
 *     or page-locked host memory through its device mapping
 *     (hipHostGetDevicePointer), which they then read and write in place
 *     over the host link (the C++ trait mirror passes large host tensors so);
 *   - enqueues its kernels on that stream and returns without synchronizing;
 *   - never allocates or frees memory (all buffers are caller-owned and must
 *     outlive the queued work);
 *   - returns SPH_OK (0) or a negative status; sph_status_string() names it.
 * Functions are reentrant and hold no per-call state; ordering is per stream.
 *
 * Numerics: every op computes in f32 from inputs widened exactly (f16/bf16
 * → f32), as the reference's CPU kernels do; half-precision outputs are the
 * f32 result rounded once, to nearest-even.
 *
 * Citations name the reference interface each entry point replaces
 * (paths relative to the sapient workspace root).
 */
#ifndef SAPIENT_HIP_H
#define SAPIENT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPH_ABI_VERSION 1

/* Status codes. */
#define SPH_OK 0
#define SPH_EINVAL (-1)  /* null pointer, unsupported dtype, bad shape or alignment */
#define SPH_EHIP (-2)    /* the HIP runtime reported an error while enqueueing */
#define SPH_ERANGE (-3)  /* a token id is outside [0, vocab), or cache positions past max_seq */
#define SPH_ENODEV (-4)  /* no usable gfx950 device is current */
#define SPH_ESTATE (-5)  /* one-time set-up cannot run now: the stream is being captured (call sph_init first) */

/* Element / table types, numbered as GGUF tensor type ids
 * (crates/sapient-io/src/gguf.rs:90-104). That enum is private to the
 * reference's loader, so a caller maps its own dtype enum
 * (sapient_core::DType, crates/sapient-core/src/dtype.rs:16) to these codes. */
#define SPH_F32 0
#define SPH_F16 1
#define SPH_Q4_0 2
#define SPH_Q8_0 8
#define SPH_Q4_K 12
#define SPH_Q5_K 13
#define SPH_Q6_K 14
#define SPH_BF16 30

/* RoPE pair layouts. */
#define SPH_ROPE_NEOX 0        /* rotate_half: pairs (i, i + rotary_dim/2) */
#define SPH_ROPE_INTERLEAVED 1 /* ggml NORM: pairs (2i, 2i + 1) */

/* Library identity and diagnostics. */
int sph_abi_version(void);
const char* sph_status_string(int status);

/* One-time per-device set-up (the GELU lookup tables). Optional: the first
 * half-precision sph_gelu_tanh / sph_gelu_erf call on a device does it lazily;
 * call it first when later calls will be captured into a HIP graph (a lazy
 * set-up under capture returns SPH_ESTATE and enqueues nothing). Synchronizes
 * `stream` once. */
int sph_init(void* stream);

/* RMSNorm over the last dimension, `rows` rows of `dim` elements:
 *   y = x * (1 / sqrt(mean(x^2) + eps)) * weight.
 * Replaces LlmBackend::rms_norm (crates/sapient-models/src/forward/backend.rs:72)
 * → kernels::layernorm::rms_norm (crates/sapient-backends/cpu/src/kernels/layernorm.rs:75-106),
 * and the wgpu analog WgpuContext::rms_norm (crates/sapient-backends/wgpu/src/resident.rs:237).
 * x_dtype ∈ {F32, F16, BF16}; w_dtype ∈ {F32, x_dtype}; out_dtype ∈ {F32, x_dtype}.
 * `weight` may be NULL (unit weight, as the kernel's Option<&Tensor>). */
int sph_rms_norm(const void* x, int x_dtype, const void* weight, int w_dtype, void* out,
                 int out_dtype, int64_t rows, int64_t dim, float eps, void* stream);

/* Fused residual add + RMSNorm: r = x + residual (written back into
 * `residual`, rounded to `dtype`), out = rms_norm(r) computed from the f32 sum.
 * Replaces the pair LlmBackend::add → LlmBackend::rms_norm
 * (crates/sapient-models/src/forward/llama.rs:508 then :515; wgpu analog
 * crates/sapient-models/src/forward/wgpu_engine.rs:469 then :472).
 * dtype ∈ {F32, F16, BF16} for x and residual; w_dtype ∈ {F32, dtype};
 * out_dtype ∈ {F32, dtype}. `out` must not alias x or residual. */
int sph_add_rms_norm(const void* x, void* residual, int dtype, const void* weight, int w_dtype,
                     void* out, int out_dtype, int64_t rows, int64_t dim, float eps, void* stream);

/* sph_add_rms_norm with the sum written to `sum` and `residual` only read:
 * the pair as the trait returns it, LlmBackend::add producing a new tensor
 * (crates/sapient-backends/cpu/src/kernels/elementwise.rs:27-57, called at
 * llama.rs:508) that LlmBackend::rms_norm then reads (:515). For callers whose
 * inputs must survive the call (host-tensor backends, whose kernels can then
 * read and write host memory in place). sum == residual is sph_add_rms_norm;
 * otherwise `sum` must not alias x, and `out` none of x, residual and sum.
 * The sum is sph_add_rms_norm's bit for bit; so is `out` when sum and
 * residual share their 16-byte alignment (the launch shape follows the
 * pointers' alignment, and shapes differ only in the order of a row's sum of
 * squares). */
int sph_add_rms_norm_to(const void* x, const void* residual, void* sum, int dtype, const void* weight,
                        int w_dtype, void* out, int out_dtype, int64_t rows, int64_t dim, float eps,
                        void* stream);

/* LayerNorm over the last dimension, two-pass mean then variance:
 *   mean = sum(x) / dim;  var = sum((x - mean)^2) / dim;
 *   y = ((x - mean) * (1 / sqrt(var + eps))) * weight + bias.
 * Replaces LlmBackend::layer_norm (backend.rs:73-79) → common::layer_norm
 * (crates/sapient-models/src/forward/common.rs:575-577) → kernels::layernorm::layer_norm
 * (layernorm.rs:17-69, axis = -1), and the wgpu analog WgpuContext::layer_norm
 * (resident.rs:277). `weight` and `bias` may each be NULL (the kernel's
 * Option<&Tensor> cases, layernorm.rs:59-64); both are of wb_dtype ∈ {F32, x_dtype}.
 * x_dtype ∈ {F32, F16, BF16}; out_dtype ∈ {F32, x_dtype}. */
int sph_layer_norm(const void* x, int x_dtype, const void* weight, const void* bias, int wb_dtype,
                   void* out, int out_dtype, int64_t rows, int64_t dim, float eps, void* stream);

/* Element-wise a + b and a * b with the reference's broadcast rule: same
 * length, or either operand of length 1 (elementwise.rs:27-57, :61-69).
 * Replaces LlmBackend::add / LlmBackend::mul (backend.rs:82-83). `out` has
 * max(na, nb) elements and may alias a full-length input. */
int sph_add(const void* a, int64_t na, const void* b, int64_t nb, void* out, int dtype, void* stream);
int sph_mul(const void* a, int64_t na, const void* b, int64_t nb, void* out, int dtype, void* stream);

/* SiLU: x / (1 + exp(-x)). Replaces LlmBackend::silu (backend.rs:80)
 * → elementwise::silu (crates/sapient-backends/cpu/src/kernels/elementwise.rs:141-143).
 * Bit-exact with the reference on glibc in every dtype (half outputs: the
 * reference's f32 result rounded once): exp is evaluated by glibc's own expf
 * algorithm wherever it can change the result. */
int sph_silu(const void* x, void* out, int dtype, int64_t n, void* stream);

/* SwiGLU: silu(gate) * up, fused. Replaces LlmBackend::silu then ::mul
 * (llama.rs:531-532) and the wgpu analog WgpuContext::swiglu (resident.rs:409).
 * Bit-exact like sph_silu. `out` may alias `gate` or `up`. */
int sph_swiglu(const void* gate, const void* up, void* out, int dtype, int64_t n, void* stream);

/* GELU, tanh approximation: 0.5 x (1 + tanh(0.79788456 (x + 0.044715 x^3))).
 * Replaces LlmBackend::gelu (backend.rs:81) → elementwise::gelu
 * (elementwise.rs:120-127). Bit-exact with the reference on glibc: tanh is
 * evaluated by glibc's own tanhf algorithm. `out` may alias `x`. */
int sph_gelu_tanh(const void* x, void* out, int dtype, int64_t n, void* stream);

/* Exact-form GELU: 0.5 x (1 + erf(x / sqrt(2))), erf by the reference's
 * Abramowitz-Stegun rational approximation with glibc's expf.
 * Replaces elementwise::gelu_erf (elementwise.rs:135-138, erf_approx :163-174)
 * and WgpuContext::gelu_erf (resident.rs:316). Bit-exact with the reference
 * on glibc. `out` may alias `x`. */
int sph_gelu_erf(const void* x, void* out, int dtype, int64_t n, void* stream);

/* Bias over the last dimension: out[i] = y[i] + bias[i % n], `total` elements
 * of y, a multiple of n. Replaces common::add_bias_last_dim
 * (crates/sapient-models/src/forward/common.rs:556-569, the bias step of
 * LlmBackend::linear_3d_bias, backend.rs:64-70) and WgpuContext::add_bias
 * (resident.rs:416). dtype ∈ {F32, F16, BF16} for y and out;
 * bias_dtype ∈ {F32, dtype}. `out` may alias `y`. */
int sph_add_bias(const void* y, const void* bias, int bias_dtype, void* out, int dtype, int64_t total, int64_t n,
                 void* stream);

/* Rotary position embedding, in place, on up to two tensors sharing positions
 * (Q and K). Each tensor is [batch, heads, seq, head_dim] contiguous (the
 * reference's rank-4 layout, rope.rs:18-26). Channels [0, rotary_dim) rotate,
 * the rest pass through; the angle of pair i at position p is
 *   (p / pos_scale) / powf(base, 2i / rotary_dim).
 * Replaces LlmBackend::apply_rope_positions (backend.rs:84) → rope::apply_rope
 * (crates/sapient-backends/cpu/src/kernels/rope.rs:18-62, rotary_dim = head_dim,
 * pos_scale = 1), LlmBackend::apply_rope_partial (backend.rs:89-97) →
 * rope::apply_rope_partial_scaled (rope.rs:83-136), and WgpuContext::rope
 * (resident.rs:467). layout = SPH_ROPE_INTERLEAVED rotates (2i, 2i+1) pairs
 * instead (the layout the reference reaches by permuting GGUF q/k rows,
 * crates/sapient-models/src/gguf_weights.rs:111-115). Bit-exact with the
 * reference on glibc: powf from the host libm, sinf/cosf by glibc's algorithm.
 * `k` may be NULL (n_k_heads ignored). positions: device int32[seq], >= 0.
 * dtype ∈ {F32, F16, BF16}; head_dim even; rotary_dim even, 2..min(head_dim, 512). */
int sph_rope(void* q, int64_t n_q_heads, void* k, int64_t n_k_heads, int dtype, int layout,
             const int32_t* positions, int64_t batch, int64_t seq, int64_t head_dim,
             int64_t rotary_dim, float base, float pos_scale, void* stream);

/* sph_rope with the angles read from tables instead of evaluated on the device:
 * cos_table / sin_table are device f32 [table_rows, rotary_dim / 2] (4-byte
 * aligned), row r holding cos / sin of row r's angle for each pair — the
 * layout of rope::rope_cos_sin_cache (crates/sapient-backends/cpu/src/kernels/rope.rs:140-153),
 * which sph_rope_table fills on the host. Token s reads row positions[s]
 * (device int32[seq]), or row s when `positions` is NULL (tables built for
 * this call's positions; then table_rows >= seq, else SPH_ERANGE). A row
 * outside [0, table_rows) leaves that token's channels unchanged and stores 1
 * to `bad_pos_flag` (device int32, optional). Replaces
 * LlmBackend::apply_rope_positions / apply_rope_partial / apply_rope_interleaved
 * (crates/sapient-models/src/forward/backend.rs:84-97), whose positions are on
 * the host (`positions: &[usize]`) and whose angles the reference evaluates
 * with host libm (rope.rs:49-50, :123-125): with tables from sph_rope_table
 * the result is sph_rope's, bit for bit, and the kernel evaluates no sin/cos.
 * Other arguments and rules are sph_rope's (base and pos_scale are in the tables). */
int sph_rope_cached(void* q, int64_t n_q_heads, void* k, int64_t n_k_heads, int dtype, int layout,
                    const float* cos_table, const float* sin_table, int64_t table_rows,
                    const int32_t* positions, int64_t batch, int64_t seq, int64_t head_dim,
                    int64_t rotary_dim, int32_t* bad_pos_flag, void* stream);

/* Host function (no device work): fill HOST arrays cos_out / sin_out
 * [n, rotary_dim / 2] with the RoPE angles of n positions, row r for
 * positions[r] (or r when `positions` is NULL): the reference's
 *   freq = (pos as f32 / pos_scale) / base.powf(2i / rotary_dim)
 * (rope.rs:48-50, :123-125) and its sin / cos, by the host libm the
 * reference's f32::powf / f32::sin_cos call. positions NULL, rotary_dim =
 * head_dim and pos_scale = 1 give rope::rope_cos_sin_cache(n, head_dim, base)
 * (rope.rs:140-153). Negative positions, odd rotary_dim or pos_scale 0 / NaN:
 * SPH_EINVAL. */
int sph_rope_table(const int64_t* positions, int64_t n, int64_t rotary_dim, float base, float pos_scale,
                   float* cos_out, float* sin_out);

/* Decode-step fusion of RoPE and the KV-cache append: q [n_q_heads, seq,
 * head_dim] is rotated in place; k and v [n_kv_heads, seq, head_dim] are read
 * (not modified), and for each token s the rotated k row and the v row are
 * written to kcache / vcache [n_kv_heads, max_seq, head_dim] at row
 * positions[s], converted to cache_dtype (nearest-even for half caches).
 * Results equal sph_rope (batch 1, rotary_dim = head_dim) on q and k followed
 * by sph_kv_append of k and v at pos = positions[0] when positions are
 * consecutive — the sequence of WgpuForwardEngine::forward_token
 * (crates/sapient-models/src/forward/wgpu_engine.rs:408-432, resident.rs:467
 * then :645-711) — in one launch. Positions are read on the device, so a HIP
 * graph capturing this call replays correctly as positions change. A position
 * outside [0, max_seq) writes nothing to the caches and stores 1 to
 * `bad_pos_flag` (device int32, optional). dtype ∈ {F32, F16, BF16} for q, k,
 * v; cache_dtype ∈ {F32, F16, BF16}; head_dim even, ≤ 512, and such that the
 * rows allow 16-byte-or-narrower vector access (any multiple of 8 does).
 * Optional biases bq [n_q_heads · head_dim], bk and bv [n_kv_heads · head_dim]
 * (bias_dtype ∈ {F32, F16, BF16}; NULL = none) are added first, as
 * sph_add_bias on q, k, v would (the projections' bias step,
 * wgpu_engine.rs:397-407): the sum is rounded to `dtype` before RoPE / the
 * cache conversion, so the result equals that unfused sequence bit for bit. */
int sph_rope_kv_append(void* q, int64_t n_q_heads, const void* k, const void* v, int64_t n_kv_heads, int dtype,
                       int layout, const int32_t* positions, int64_t seq, int64_t head_dim, float base,
                       float pos_scale, void* kcache, void* vcache, int cache_dtype, int64_t max_seq,
                       const void* bq, const void* bk, const void* bv, int bias_dtype, int32_t* bad_pos_flag,
                       void* stream);

/* sph_rope_kv_append for a chunk straight from the projections: q, k and v
 * are read token-major, [seq, n_q_heads | n_kv_heads, head_dim] (not
 * modified), and the rotated q is written heads-major to q_out [n_q_heads,
 * seq, head_dim], the layout attention reads. Replaces the chunk sequence of
 * WgpuForwardEngine::forward_chunk (wgpu_engine.rs:525-573): bias adds,
 * transpose_heads of q, k and v (resident.rs:420-458), rope of q and k, and
 * kv_append of k and v. Results equal sph_transpose_heads of q, k, v followed
 * by sph_rope_kv_append, bit for bit. q_out must not overlap q (SPH_EINVAL);
 * every other rule is sph_rope_kv_append's. */
int sph_rope_kv_append_tokens(const void* q, void* q_out, int64_t n_q_heads, const void* k, const void* v,
                              int64_t n_kv_heads, int dtype, int layout, const int32_t* positions, int64_t seq,
                              int64_t head_dim, float base, float pos_scale, void* kcache, void* vcache,
                              int cache_dtype, int64_t max_seq, const void* bq, const void* bk, const void* bv,
                              int bias_dtype, int32_t* bad_pos_flag, void* stream);

/* Token-embedding gather with on-the-fly row dequantization into f32:
 * out[t, :] = dequant(table[ids[t], :]). The table is the raw GGUF tensor
 * data, rows of byte_count(hidden) bytes, consumed verbatim (no repacking).
 * Replaces common::embed_tokens (crates/sapient-models/src/forward/common.rs:164-217)
 * and WgpuContext::embed / embed_q8_0 / embed_q4_k (resident.rs:714,
 * quant.rs:445, quant.rs:273). table_dtype ∈ {F32, F16, BF16, Q4_0, Q8_0, Q4_K,
 * Q5_K, Q6_K} — every type gather_row_f32 accepts (common.rs:186-214; the
 * row-interleaved R4 repacks are refused there too);
 * hidden a multiple of the block width (32 for Q4_0 / Q8_0, 256 for K-quants).
 * ids: device uint32[n_ids]. An id >= vocab never reads the table: its
 * output row is zero-filled and, if `bad_id_flag` (device int32) is not NULL,
 * 1 is stored there. Callers holding the ids on the host validate them first,
 * as the reference does (common.rs:171-173). */
int sph_embed(const void* table, int table_dtype, int64_t vocab, int64_t hidden,
              const uint32_t* ids, int64_t n_ids, float* out, int32_t* bad_id_flag, void* stream);

/* Swap the two leading axes: x [outer, inner, head_dim] → out [inner, outer,
 * head_dim], head_dim-element rows moving as units (the matmul layout
 * [seq, heads, hd] ↔ the attention layout [heads, seq, hd]). Replaces
 * WgpuContext::transpose_heads (crates/sapient-backends/wgpu/src/resident.rs:420-458).
 * dtype ∈ {F32, F16, BF16}; elements are moved bit for bit. `out` must not
 * overlap `x`. outer · inner < 2^32. */
int sph_transpose_heads(const void* x, void* out, int dtype, int64_t outer, int64_t inner, int64_t head_dim,
                        void* stream);

/* KV-cache append: src [n_kv, seq, head_dim] (heads-major) is written to
 * positions pos .. pos+seq-1 of cache [n_kv, max_seq, head_dim], converted to
 * the cache's type (f32 → f16 / bf16 rounds to nearest-even). seq = 1 is a
 * decode step, seq > 1 a batched prefill. Replaces WgpuContext::kv_append
 * (resident.rs:645-711). src_dtype ∈ {F32, F16, BF16}; cache_dtype ∈ {F32,
 * F16, BF16, Q8_0}. A Q8_0 cache is the reference's quantized KV cache
 * (update_kv_cache_q8, crates/sapient-models/src/forward/common.rs:449-508):
 * rows of head_dim / 32 blocks of 34 bytes (f16 scale, 32 × i8), each block
 * quantized on append as quantize_f32_to_q8_0_block does (common.rs:336-348),
 * bit for bit; head_dim a multiple of 32, src 16-byte and cache 2-byte
 * aligned. pos + seq > max_seq returns SPH_ERANGE without writing. */
int sph_kv_append(const void* src, int src_dtype, void* cache, int cache_dtype, int64_t n_kv, int64_t seq,
                  int64_t head_dim, int64_t max_seq, int64_t pos, void* stream);

/* The trait path's KV-cache update, sliding window included. Replaces
 * common::update_kv_cache (crates/sapient-models/src/forward/common.rs:355-434,
 * called at llama.rs:489-490 and phi.rs:461-462) and its Q8_0 cache,
 * update_kv_cache_q8 (:449-508). cache [n_kv, max_seq, head_dim] (the
 * reference's [batch, heads, max_seq, head_dim] with batch · heads folded into
 * n_kv) holds cur_len valid rows per head; src [n_kv, seq, head_dim] is
 * appended after them. When cur_len + seq > max_seq the oldest
 * shift = cur_len + seq - max_seq rows of every head are dropped first (rows
 * [shift, cur_len) move to [0, cur_len - shift), common.rs:392-405) and src
 * lands at cur_len - shift. *new_len (host int64) receives min(cur_len + seq,
 * max_seq), the length of the view the reference returns. seq > max_seq
 * returns SPH_ERANGE (the reference's "new tokens exceeds max cache size"),
 * cur_len > max_seq SPH_EINVAL; nothing is written then, nor when the append
 * itself would be rejected (its checks run before the shift). Types,
 * conversion and the Q8_0 layout are sph_kv_append's. The shift runs as two
 * in-place row-reversal passes (one launch each for n_kv <= 65535, more for
 * larger n_kv) and the append as one launch (more past 2^31 work items); the
 * rows moved by the shift are copied bit for bit, and the shift's rows past
 * cur_len - shift hold intermediate values until the append overwrites them.
 * The in-place shift moves every kept row twice; sph_kv_cache_update_into
 * moves it once, into a second buffer. */
int sph_kv_cache_update(const void* src, int src_dtype, void* cache, int cache_dtype, int64_t n_kv, int64_t seq,
                        int64_t head_dim, int64_t max_seq, int64_t cur_len, int64_t* new_len, void* stream);

/* sph_kv_cache_update into a second, caller-owned cache: `out` (same layout
 * and type as `cache`) receives the updated cache — rows [0, *new_len) of
 * every head: the kept rows cache[shift .. cur_len), then src converted to
 * the cache type — and `cache` is only read. Rows of `out` past *new_len are
 * left as they were. Replaces common::update_kv_cache / update_kv_cache_q8
 * (crates/sapient-models/src/forward/common.rs:355-434, :449-508) for a
 * caller that then replaces its cache tensor with `out`, which the reference's
 * signature allows: it takes the cache as `&mut Tensor` (:355-359, :449-455).
 * Each kept row crosses HBM once each way, and a float cache
 * whose rows split into 16-byte units (16-byte aligned buffers) takes a
 * single launch for the move and the append; other rows take two (the
 * move as raw units, then sph_kv_append). Results equal sph_kv_cache_update's
 * rows [0, *new_len) bit for bit. When no row is dropped (cur_len + seq <=
 * max_seq) this still copies the cur_len rows: such a step is cheaper in
 * place. Arguments and errors are sph_kv_cache_update's; `out` must not
 * overlap `cache` or `src` (SPH_EINVAL). */
int sph_kv_cache_update_into(const void* src, int src_dtype, const void* cache, void* out, int cache_dtype,
                             int64_t n_kv, int64_t seq, int64_t head_dim, int64_t max_seq, int64_t cur_len,
                             int64_t* new_len, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SAPIENT_HIP_H */
