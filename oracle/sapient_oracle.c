/*
 * sapient_oracle.c — CPU oracle for the fused per-layer op set.
 *
 * TEST INFRASTRUCTURE ONLY. This file is a plain-C restatement of the
 * reference's scalar Rust CPU kernels. Only the test suite, the smoke check
 * and the benchmark's CPU-baseline leg load it (as liboracle.so through
 * ctypes); the product library never links or calls it.
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math, linked against glibc libm.
 * Rust's f32::{exp,tanh,powf,sin,cos} bind to the same libm functions
 * (expf, tanhf, powf, sinf, cosf) on x86_64-linux-gnu, Rust never contracts
 * a*b+c into an FMA, and Iterator::sum::<f32>() is a left-to-right fold, so
 * every loop below keeps the reference's operation order and rounding points.
 *
 * Each function names the reference file:line it follows (paths relative to
 * the sapient workspace root). Functions whose results no reference test,
 * closed form or independent restatement pins are marked "parity unpinned";
 * there are none at present (see the tests under tests/).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define SOR_OK 0
#define SOR_EINVAL (-1)
#define SOR_ERANGE (-3)

/* Table dtypes for the embedding gather: GGUF type ids (crates/sapient-io/src/gguf.rs:90-104). */
enum { SOR_F32 = 0, SOR_F16 = 1, SOR_Q4_0 = 2, SOR_Q8_0 = 8, SOR_Q4_K = 12, SOR_Q5_K = 13, SOR_Q6_K = 14, SOR_BF16 = 30 };

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ───────────────────────── half-precision conversions ─────────────────────────
 * The reference widens with crate `half` 2.7.1 (tensor.rs:348-361,
 * common.rs:192-203); widening is exact, NaNs come out quiet. Narrowing (the outputs the HIP
 * library stores as f16/bf16) follows half's from_f32: IEEE round-to-nearest-even,
 * NaN kept quiet with the top mantissa bits. */

float sor_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0x1F) return u2f(sign | 0x7F800000u | (man ? 0x400000u | (man << 13) : 0u)); /* NaN: quiet bit set, as half does */
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal half: value = man * 2^-24, exact in f32 */
        float v = (float)man * 0x1p-24f;
        return sign ? -v : v;
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t sor_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) {
        if (man == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7C00u | 0x200u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign; /* below half the smallest subnormal */
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_m = m >> shift;
        uint32_t rbit = 1u << (shift - 1);
        uint32_t rest = m & ((rbit << 1) - 1u);
        if ((m & rbit) && ((rest & (rbit - 1u)) || (half_m & 1u))) half_m += 1u;
        return (uint16_t)(sign | half_m);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rbit = 0x1000u;
    if ((man & rbit) && (man & (3u * rbit - 1u))) h += 1u; /* carries into exp/inf correctly */
    return (uint16_t)h;
}

float sor_bf16_to_f32(uint16_t h) {
    if ((h & 0x7FFFu) > 0x7F80u) h |= 0x40u; /* NaN: quiet bit set, as half does */
    return u2f((uint32_t)h << 16);
}

uint16_t sor_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t rbit = 0x8000u;
    if ((x & rbit) && (x & (3u * rbit - 1u))) return (uint16_t)((x >> 16) + 1u);
    return (uint16_t)(x >> 16);
}

void sor_f16_to_f32_n(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = sor_f16_to_f32(in[i]);
}
void sor_f32_to_f16_n(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = sor_f32_to_f16(in[i]);
}
void sor_bf16_to_f32_n(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = sor_bf16_to_f32(in[i]);
}
void sor_f32_to_bf16_n(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = sor_f32_to_bf16(in[i]);
}

/* ───────────────────────────── a1: RMSNorm ─────────────────────────────
 * crates/sapient-backends/cpu/src/kernels/layernorm.rs:75-106
 *   rms_sq  = (Σ_serial v*v) / dim            (:97)
 *   inv_rms = 1.0 / sqrt(rms_sq + eps)        (:98)
 *   out[i]  = x[i] * inv_rms * w[i]           (:101, left to right)
 * `weight` may be NULL (the reference's `w.map_or(1.0, ..)`). */
void sor_rms_norm(const float* x, const float* w, float* out, size_t outer, size_t dim, float eps) {
    for (size_t o = 0; o < outer; o++) {
        const float* row = x + o * dim;
        float acc = -0.0f; /* Sum for f32 folds from -0.0; x*x >= 0 so the start value never shows */
        for (size_t i = 0; i < dim; i++) acc = acc + row[i] * row[i];
        float rms_sq = acc / (float)dim;
        float inv = 1.0f / sqrtf(rms_sq + eps);
        for (size_t i = 0; i < dim; i++) {
            float t = row[i] * inv;
            out[o * dim + i] = w ? t * w[i] : t * 1.0f;
        }
    }
}

/* ─────────────────────── next row f3: LayerNorm, bias add ───────────────────────
 * crates/sapient-backends/cpu/src/kernels/layernorm.rs:17-69 (axis = -1, as
 * common::layer_norm calls it, common.rs:575-577):
 *   mean = (Σ_serial v) / n;  var = (Σ_serial (v-mean)*(v-mean)) / n
 *   inv_std = 1 / sqrt(var + eps);  normed = (x - mean) * inv_std
 *   out = normed * w + b  (each of w, b optional; two roundings, no FMA) */
void sor_layer_norm(const float* x, const float* w, const float* b, float* out, size_t outer, size_t n, float eps) {
    for (size_t o = 0; o < outer; o++) {
        const float* row = x + o * n;
        float s = -0.0f;
        for (size_t i = 0; i < n; i++) s = s + row[i];
        float mean = s / (float)n;
        float v = -0.0f;
        for (size_t i = 0; i < n; i++) v = v + (row[i] - mean) * (row[i] - mean);
        float var = v / (float)n;
        float inv_std = 1.0f / sqrtf(var + eps);
        for (size_t i = 0; i < n; i++) {
            float normed = (row[i] - mean) * inv_std;
            float y = normed;
            if (w && b) y = normed * w[i] + b[i];
            else if (w) y = normed * w[i];
            else if (b) y = normed + b[i];
            out[o * n + i] = y;
        }
    }
}

/* crates/sapient-models/src/forward/common.rs:556-569 (add_bias_last_dim):
 * y [.., n] f32, bias [n] (any float dtype, widened): out[k] = y[k] + b[k % n]. */
void sor_add_bias_last_dim(const float* y, const float* bias, float* out, size_t total, size_t n) {
    for (size_t k = 0; k < total; k++) out[k] = y[k] + bias[k % n];
}

/* ─────────────────────── a2: residual add, mul ───────────────────────
 * crates/sapient-backends/cpu/src/kernels/elementwise.rs:61-63 (add), :67-69 (mul),
 * through binary_f32 :27-57: same length, or either side of length 1 broadcast.
 * Returns SOR_EINVAL for the reference's ShapeMismatch. */
static int binary(const float* a, size_t na, const float* b, size_t nb, float* out, int op) {
    if (na == nb) {
        for (size_t i = 0; i < na; i++) out[i] = op ? a[i] * b[i] : a[i] + b[i];
    } else if (nb == 1) {
        for (size_t i = 0; i < na; i++) out[i] = op ? a[i] * b[0] : a[i] + b[0];
    } else if (na == 1) {
        for (size_t i = 0; i < nb; i++) out[i] = op ? a[0] * b[i] : a[0] + b[i];
    } else {
        return SOR_EINVAL;
    }
    return SOR_OK;
}
int sor_add(const float* a, size_t na, const float* b, size_t nb, float* out) { return binary(a, na, b, nb, out, 0); }
int sor_mul(const float* a, size_t na, const float* b, size_t nb, float* out) { return binary(a, na, b, nb, out, 1); }

/* Fused residual add + RMSNorm. The reference has no fused op: it runs
 * `bk.add` (crates/sapient-models/src/forward/llama.rs:508) and then
 * `bk.rms_norm` on the sum (llama.rs:515). Outputs (normed, updated residual). */
void sor_add_rms_norm(const float* x, const float* residual, const float* w, float* normed,
                      float* residual_out, size_t rows, size_t dim, float eps) {
    size_t n = rows * dim;
    for (size_t i = 0; i < n; i++) residual_out[i] = x[i] + residual[i];
    sor_rms_norm(residual_out, w, normed, rows, dim, eps);
}

/* ───────────────────────── a3: SiLU and SwiGLU ─────────────────────────
 * elementwise.rs:141-143  silu(v) = v / (1.0 + exp(-v))   (glibc expf)
 * SwiGLU = silu(gate) then mul(up): llama.rs:531-532 → elementwise.rs:67-69. */
void sor_silu(const float* x, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        out[i] = v / (1.0f + expf(-v));
    }
}
void sor_swiglu(const float* gate, const float* up, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float v = gate[i];
        float s = v / (1.0f + expf(-v));
        out[i] = s * up[i];
    }
}

/* ───────────────────────────── a4: GELU (tanh) ─────────────────────────────
 * elementwise.rs:120-127
 *   inner = 0.797_884_56 * (v + 0.044_715 * v * v * v)
 *   y     = 0.5 * v * (1.0 + tanh(inner))               (glibc tanhf) */
void sor_gelu(const float* x, float* out, size_t n) {
    const float S = 0.79788456f, C = 0.044715f;
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        float inner = S * (v + C * v * v * v);
        out[i] = 0.5f * v * (1.0f + tanhf(inner));
    }
}

/* erf-GELU (next row): elementwise.rs:135-138 with erf_approx :163-174. */
static float erf_approx(float x) {
    float sign = (x > 0.0f) ? 1.0f : (x < 0.0f ? -1.0f : (signbit(x) ? -1.0f : 1.0f));
    if (isnan(x)) sign = x;
    x = fabsf(x);
    float t = 1.0f / (1.0f + 0.3275911f * x);
    float y = 1.0f - (0.25482959f + (-0.28449674f + (1.42141374f + (-1.45315203f + 1.06140543f * t) * t) * t) * t) * t * expf(-x * x);
    return sign * y;
}
void sor_gelu_erf(const float* x, float* out, size_t n) {
    const float INV_SQRT_2 = 0.70710678118654752440f;
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        out[i] = 0.5f * v * (1.0f + erf_approx(v * INV_SQRT_2));
    }
}

/* ───────────────────────────── a5: RoPE (NEOX) ─────────────────────────────
 * crates/sapient-backends/cpu/src/kernels/rope.rs:18-62 (apply_rope):
 *   x is [batch, n_heads, seq_len, head_dim] (rank 4, :19-26), head_dim even
 *   (:28-30), positions.len() == seq_len (:31-35); for i < head_dim/2:
 *     freq = (pos as f32) / base.powf(2.0 * i as f32 / head_dim as f32)   (:49)
 *     (sin, cos) = freq.sin_cos()                                         (:50)
 *     o[i]        = x0 * cos - x1 * sin                                   (:56)
 *     o[i + half] = x1 * cos + x0 * sin                                   (:57)
 * Out of place: `out` starts as a copy of x (:40). */
int sor_apply_rope(const float* x, float* out, size_t batch, size_t n_heads, size_t seq_len,
                   size_t head_dim, const int64_t* positions, size_t n_positions, float base) {
    if (head_dim % 2 != 0) return SOR_EINVAL;
    if (n_positions != seq_len) return SOR_EINVAL;
    size_t half = head_dim / 2;
    size_t n = batch * n_heads * seq_len * head_dim;
    memmove(out, x, n * sizeof(float));
    for (size_t b = 0; b < batch; b++)
        for (size_t h = 0; h < n_heads; h++)
            for (size_t s = 0; s < seq_len; s++) {
                size_t base_idx = ((b * n_heads + h) * seq_len + s) * head_dim;
                for (size_t i = 0; i < half; i++) {
                    float freq = (float)positions[s] / powf(base, 2.0f * (float)i / (float)head_dim);
                    float sn = sinf(freq), cs = cosf(freq);
                    float x0 = x[base_idx + i], x1 = x[base_idx + i + half];
                    out[base_idx + i] = x0 * cs - x1 * sn;
                    out[base_idx + i + half] = x1 * cs + x0 * sn;
                }
            }
    return SOR_OK;
}

/* rope.rs:83-136 (apply_rope_partial_scaled; apply_rope_partial is pos_scale = 1):
 *   1 <= rotary_dim <= head_dim, rotary_dim even (:99-104)
 *   freq = (pos as f32 / pos_scale) / base.powf(2.0 * i as f32 / rotary_dim as f32)  (:123-124)
 *   channels [rotary_dim, head_dim) pass through. */
int sor_apply_rope_partial_scaled(const float* x, float* out, size_t batch, size_t n_heads,
                                  size_t seq_len, size_t head_dim, const int64_t* positions,
                                  size_t n_positions, float base, size_t rotary_dim, float pos_scale) {
    if (rotary_dim == 0 || rotary_dim > head_dim) return SOR_EINVAL;
    if (rotary_dim % 2 != 0) return SOR_EINVAL;
    if (n_positions != seq_len) return SOR_EINVAL;
    size_t half = rotary_dim / 2;
    size_t n = batch * n_heads * seq_len * head_dim;
    memmove(out, x, n * sizeof(float));
    for (size_t b = 0; b < batch; b++)
        for (size_t h = 0; h < n_heads; h++)
            for (size_t s = 0; s < seq_len; s++) {
                size_t base_idx = ((b * n_heads + h) * seq_len + s) * head_dim;
                for (size_t i = 0; i < half; i++) {
                    float freq = ((float)positions[s] / pos_scale) /
                                 powf(base, 2.0f * (float)i / (float)rotary_dim);
                    float sn = sinf(freq), cs = cosf(freq);
                    float x0 = x[base_idx + i], x1 = x[base_idx + i + half];
                    out[base_idx + i] = x0 * cs - x1 * sn;
                    out[base_idx + i + half] = x1 * cs + x0 * sn;
                }
            }
    return SOR_OK;
}

/* ─────────────────────────── a6: RoPE (interleaved) ───────────────────────────
 * No reference function: the reference un-permutes GGUF q/k rows at load so
 * that its NEOX RoPE applies (crates/sapient-models/src/gguf_weights.rs:111-115:
 * HF row h·D + a·D/2 + b  ↔  GGUF row h·D + 2b + a). Rotating pairs
 * (x[2i], x[2i+1]) with the NEOX frequency of index i is the operator that
 * satisfies interleaved(P·x) = P·neox(x) for that permutation P; the tests pin
 * this identity against sor_apply_rope_partial_scaled bit for bit. */
int sor_apply_rope_interleaved(const float* x, float* out, size_t batch, size_t n_heads,
                               size_t seq_len, size_t head_dim, const int64_t* positions,
                               size_t n_positions, float base, size_t rotary_dim, float pos_scale) {
    if (rotary_dim == 0 || rotary_dim > head_dim) return SOR_EINVAL;
    if (rotary_dim % 2 != 0) return SOR_EINVAL;
    if (n_positions != seq_len) return SOR_EINVAL;
    size_t half = rotary_dim / 2;
    size_t n = batch * n_heads * seq_len * head_dim;
    memmove(out, x, n * sizeof(float));
    for (size_t b = 0; b < batch; b++)
        for (size_t h = 0; h < n_heads; h++)
            for (size_t s = 0; s < seq_len; s++) {
                size_t base_idx = ((b * n_heads + h) * seq_len + s) * head_dim;
                for (size_t i = 0; i < half; i++) {
                    float freq = ((float)positions[s] / pos_scale) /
                                 powf(base, 2.0f * (float)i / (float)rotary_dim);
                    float sn = sinf(freq), cs = cosf(freq);
                    float x0 = x[base_idx + 2 * i], x1 = x[base_idx + 2 * i + 1];
                    out[base_idx + 2 * i] = x0 * cs - x1 * sn;
                    out[base_idx + 2 * i + 1] = x1 * cs + x0 * sn;
                }
            }
    return SOR_OK;
}

/* gguf_weights.rs:114-154 (unpermute_qk_rows): dst row h·D + a·D/2 + b takes
 * src row h·D + 2b + a, rows of `row_bytes` bytes. Used by the tests to check
 * the interleaved identity and the reference's own permutation KAT. */
int sor_unpermute_qk_rows(const uint8_t* src, uint8_t* dst, size_t n_head, size_t head_dim, size_t row_bytes) {
    if (head_dim < 2 || head_dim % 2 != 0) return SOR_EINVAL;
    size_t half = head_dim / 2;
    for (size_t h = 0; h < n_head; h++)
        for (size_t a = 0; a < 2; a++)
            for (size_t b = 0; b < half; b++) {
                size_t hf_row = h * head_dim + a * half + b;
                size_t gguf_row = h * head_dim + b * 2 + a;
                memcpy(dst + hf_row * row_bytes, src + gguf_row * row_bytes, row_bytes);
            }
    return SOR_OK;
}

/* ─────────────────────── a7: GGUF block dequantization ───────────────────────
 * Block constants: crates/sapient-core/src/dtype.rs:57-69; byte_count :136-145. */
#define QK 32
#define Q4_0_BYTES 18
#define Q8_0_BYTES 34
#define QK_K 256
#define Q4_K_BYTES 144
#define Q5_K_BYTES 176
#define Q6_K_BYTES 210

static inline float le_f16(const uint8_t* p) { return sor_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* tensor.rs:362-376: byte j of the 16 after d holds element j (low nibble)
 * and element j + 16 (high nibble), each minus 8, times d. */
void sor_dequant_q4_0(const uint8_t* bytes, size_t nblocks, float* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = bytes + b * Q4_0_BYTES;
        float d = le_f16(blk);
        for (size_t j = 0; j < QK / 2; j++) {
            uint8_t byte = blk[2 + j];
            int32_t lo = (int32_t)(byte & 0x0f) - 8;
            int32_t hi = (int32_t)(byte >> 4) - 8;
            out[b * QK + j] = (float)lo * d;
            out[b * QK + j + QK / 2] = (float)hi * d;
        }
    }
}

/* tensor.rs:378-389: out[32b + j] = (block[2 + j] as i8) as f32 * d. */
void sor_dequant_q8_0(const uint8_t* bytes, size_t nblocks, float* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = bytes + b * Q8_0_BYTES;
        float d = le_f16(blk);
        for (size_t j = 0; j < QK; j++) out[b * QK + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

/* tensor.rs:567-576 (get_scale_min_k4). */
static inline void scale_min_k4(size_t j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* tensor.rs:390-398 → dequant_q4_k_block :504-527. */
void sor_dequant_q4_k(const uint8_t* bytes, size_t nblocks, float* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = bytes + b * Q4_K_BYTES;
        float d = le_f16(blk), dmin = le_f16(blk + 2);
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        float* o = out + b * QK_K;
        size_t out_idx = 0, q_off = 0, is = 0;
        for (int k = 0; k < QK_K / 64; k++) {
            uint8_t sc1, m1, sc2, m2;
            scale_min_k4(is, scales, &sc1, &m1);
            float d1 = d * (float)sc1, m1v = dmin * (float)m1;
            scale_min_k4(is + 1, scales, &sc2, &m2);
            float d2 = d * (float)sc2, m2v = dmin * (float)m2;
            for (size_t l = 0; l < 32; l++) {
                o[out_idx + l] = d1 * (float)(qs[q_off + l] & 0x0F) - m1v;
                o[out_idx + l + 32] = d2 * (float)(qs[q_off + l] >> 4) - m2v;
            }
            out_idx += 64;
            q_off += 32;
            is += 2;
        }
    }
}

/* tensor.rs:421-467: as Q4_K, plus a fifth bit per element from qh[l] —
 * bit-plane u1 = 1 << 2k for the low nibbles of 64-element chunk k, u2 =
 * 2 << 2k for the high nibbles (the per-element reading the reference
 * adopted; crates/sapient-io/src/gguf.rs:391-434 still reads one qh byte per
 * chunk, but that copy is not on the embedding path, which keeps Q5_K tables
 * as blocks, gguf.rs:160-169, :658-661). */
void sor_dequant_q5_k(const uint8_t* bytes, size_t nblocks, float* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = bytes + b * Q5_K_BYTES;
        float d = le_f16(blk), dmin = le_f16(blk + 2);
        const uint8_t* scales = blk + 4;
        const uint8_t* qh = blk + 16;
        const uint8_t* ql = blk + 48;
        float* o = out + b * QK_K;
        size_t out_idx = 0, ql_off = 0, is = 0;
        uint8_t u1 = 1, u2 = 2;
        for (int k = 0; k < QK_K / 64; k++) {
            uint8_t sc1, m1, sc2, m2;
            scale_min_k4(is, scales, &sc1, &m1);
            float d1 = d * (float)sc1, m1v = dmin * (float)m1;
            scale_min_k4(is + 1, scales, &sc2, &m2);
            float d2 = d * (float)sc2, m2v = dmin * (float)m2;
            for (size_t l = 0; l < 32; l++) {
                float hi = (qh[l] & u1) ? 16.0f : 0.0f;
                o[out_idx + l] = d1 * ((float)(ql[ql_off + l] & 0x0F) + hi) - m1v;
                float hi2 = (qh[l] & u2) ? 16.0f : 0.0f;
                o[out_idx + l + 32] = d2 * ((float)(ql[ql_off + l] >> 4) + hi2) - m2v;
            }
            out_idx += 64;
            ql_off += 32;
            is += 2;
            if (is % 8 == 0) {
                u1 = 1;
                u2 = 2;
            } else {
                u1 = (uint8_t)(u1 << 2);
                u2 = (uint8_t)(u2 << 2);
            }
        }
    }
}

/* tensor.rs:468-476 → dequant_q6_k_block :534-565 (next-row dtype). */
void sor_dequant_q6_k(const uint8_t* bytes, size_t nblocks, float* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = bytes + b * Q6_K_BYTES;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const uint8_t* sc = blk + 192;
        float d = le_f16(blk + 208);
        float* o = out + b * QK_K;
        size_t out_idx = 0, ql_off = 0, qh_off = 0, sc_base = 0;
        for (int k = 0; k < QK_K / 128; k++) {
            for (size_t l = 0; l < 32; l++) {
                size_t is = l / 16;
                float q1 = (float)((int32_t)((ql[ql_off + l] & 0x0F) | ((qh[qh_off + l] & 3) << 4)) - 32);
                float q2 = (float)((int32_t)((ql[ql_off + l + 32] & 0x0F) | (((qh[qh_off + l] >> 2) & 3) << 4)) - 32);
                float q3 = (float)((int32_t)((ql[ql_off + l] >> 4) | (((qh[qh_off + l] >> 4) & 3) << 4)) - 32);
                float q4 = (float)((int32_t)((ql[ql_off + l + 32] >> 4) | (((qh[qh_off + l] >> 6) & 3) << 4)) - 32);
                o[out_idx + l] = d * (float)(int8_t)sc[sc_base + is] * q1;
                o[out_idx + l + 32] = d * (float)(int8_t)sc[sc_base + is + 2] * q2;
                o[out_idx + l + 64] = d * (float)(int8_t)sc[sc_base + is + 4] * q3;
                o[out_idx + l + 96] = d * (float)(int8_t)sc[sc_base + is + 6] * q4;
            }
            out_idx += 128;
            ql_off += 64;
            qh_off += 32;
            sc_base += 8;
        }
    }
}

/* Bytes of one `hidden`-wide row in a table of `dtype` (dtype.rs:136-145);
 * 0 for an unsupported dtype or a width that is not a whole number of blocks. */
size_t sor_row_bytes(int dtype, size_t hidden) {
    switch (dtype) {
    case SOR_F32: return hidden * 4;
    case SOR_F16:
    case SOR_BF16: return hidden * 2;
    case SOR_Q4_0: return hidden % QK ? 0 : hidden / QK * Q4_0_BYTES;
    case SOR_Q8_0: return hidden % QK ? 0 : hidden / QK * Q8_0_BYTES;
    case SOR_Q4_K: return hidden % QK_K ? 0 : hidden / QK_K * Q4_K_BYTES;
    case SOR_Q5_K: return hidden % QK_K ? 0 : hidden / QK_K * Q5_K_BYTES;
    case SOR_Q6_K: return hidden % QK_K ? 0 : hidden / QK_K * Q6_K_BYTES;
    default: return 0;
    }
}

/* crates/sapient-models/src/forward/common.rs:164-217 (embed_tokens →
 * gather_row_f32): ids >= vocab fail (:171-173) before any row is written
 * for that id; each row is dequantized on its own (:207-212), which equals
 * slicing the row out of a full-table to_f32_vec (the :678-718 test). */
int sor_embed_tokens(const uint8_t* table, int dtype, size_t vocab, size_t hidden,
                     const uint32_t* ids, size_t n_ids, float* out) {
    size_t rb = sor_row_bytes(dtype, hidden);
    if (rb == 0) return SOR_EINVAL;
    for (size_t t = 0; t < n_ids; t++) {
        if ((size_t)ids[t] >= vocab) return SOR_ERANGE;
        const uint8_t* row = table + (size_t)ids[t] * rb;
        float* dst = out + t * hidden;
        switch (dtype) {
        case SOR_F32: memcpy(dst, row, hidden * 4); break;
        case SOR_F16:
            for (size_t i = 0; i < hidden; i++) dst[i] = le_f16(row + 2 * i);
            break;
        case SOR_BF16:
            for (size_t i = 0; i < hidden; i++) dst[i] = sor_bf16_to_f32((uint16_t)(row[2 * i] | (row[2 * i + 1] << 8)));
            break;
        case SOR_Q4_0: sor_dequant_q4_0(row, hidden / QK, dst); break;
        case SOR_Q8_0: sor_dequant_q8_0(row, hidden / QK, dst); break;
        case SOR_Q4_K: sor_dequant_q4_k(row, hidden / QK_K, dst); break;
        case SOR_Q5_K: sor_dequant_q5_k(row, hidden / QK_K, dst); break;
        case SOR_Q6_K: sor_dequant_q6_k(row, hidden / QK_K, dst); break;
        }
    }
    return SOR_OK;
}

/* crates/sapient-backends/cpu/src/kernels/quant.rs:223-235 (quantize_q8_0_block),
 * used by the reference's gather test (common.rs:697) to build Q8_0 tables. */
void sor_quantize_q8_0(const float* x, size_t nblocks, uint8_t* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const float* v = x + b * QK;
        float max_abs = 0.0f;
        for (size_t i = 0; i < QK; i++) max_abs = fmaxf(max_abs, fabsf(v[i]));
        float scale = max_abs / 127.0f;
        uint16_t d = sor_f32_to_f16(scale);
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        uint8_t* o = out + b * Q8_0_BYTES;
        o[0] = (uint8_t)(d & 0xFF);
        o[1] = (uint8_t)(d >> 8);
        for (size_t i = 0; i < QK; i++) {
            float q = roundf(v[i] * inv); /* Rust f32::round: half away from zero */
            if (isnan(q)) q = 0.0f;       /* `NaN as i8` is 0 in Rust */
            if (q < -127.0f) q = -127.0f;
            if (q > 127.0f) q = 127.0f;
            o[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

/* ─────────────── device-resident decode helpers (layout moves) ───────────────
 * transpose_heads: crates/sapient-backends/wgpu/src/resident.rs:420-458 with
 * shaders/transpose_heads.wgsl — the two leading axes of [outer, inner, hd]
 * swapped, hd-element rows moved as units: out[i][o][c] = x[o][i][c]. Elements
 * are moved as raw bytes (esize 2 or 4), so any element type passes through. */
void sor_transpose_heads(const void* x, void* out, size_t esize, size_t outer, size_t inner, size_t hd) {
    const uint8_t* src = (const uint8_t*)x;
    uint8_t* dst = (uint8_t*)out;
    for (size_t o = 0; o < outer; o++)
        for (size_t i = 0; i < inner; i++)
            memcpy(dst + (i * outer + o) * hd * esize, src + (o * inner + i) * hd * esize, hd * esize);
}

/* kv_append: resident.rs:645-711 with shaders/kv_append.wgsl and
 * kv_append_f16.wgsl — src [n_kv, seq, hd] (heads-major) written to positions
 * pos..pos+seq of the cache [n_kv, max_seq, hd], converted to the cache's
 * element type: f32 as is, f16 / bf16 rounded to nearest-even (the reference
 * test's host mirror stores half::f16::from_f32(x), tests/resident.rs:365-371).
 * pos + seq > max_seq is the reference's debug assertion (:681): SOR_ERANGE. */
int sor_kv_append(const float* src, void* cache, int cache_dtype, size_t n_kv, size_t seq, size_t hd,
                  size_t max_seq, size_t pos) {
    if (pos + seq > max_seq) return SOR_ERANGE;
    if (cache_dtype == SOR_Q8_0) {
        /* The quantized KV cache of common.rs:449-508 (update_kv_cache_q8):
         * each new row is quantized block by block with
         * quantize_f32_to_q8_0_block (common.rs:336-348), the same steps as
         * quant.rs:223-235 restated in sor_quantize_q8_0; rows of a head sit at
         * (h · max_seq + position) · (hd / 32) · 34 bytes. */
        if (hd % QK != 0) return SOR_EINVAL;
        const size_t bpr = hd / QK;
        for (size_t h = 0; h < n_kv; h++)
            for (size_t s = 0; s < seq; s++)
                sor_quantize_q8_0(src + (h * seq + s) * hd, bpr,
                                  (uint8_t*)cache + (h * max_seq + pos + s) * bpr * Q8_0_BYTES);
        return SOR_OK;
    }
    if (cache_dtype != SOR_F32 && cache_dtype != SOR_F16 && cache_dtype != SOR_BF16) return SOR_EINVAL;
    for (size_t h = 0; h < n_kv; h++)
        for (size_t s = 0; s < seq; s++)
            for (size_t c = 0; c < hd; c++) {
                const float v = src[(h * seq + s) * hd + c];
                const size_t d = (h * max_seq + pos + s) * hd + c;
                if (cache_dtype == SOR_F32) ((float*)cache)[d] = v;
                else if (cache_dtype == SOR_F16) ((uint16_t*)cache)[d] = sor_f32_to_f16(v);
                else ((uint16_t*)cache)[d] = sor_f32_to_bf16(v);
            }
    return SOR_OK;
}

/* The trait path's cache update with its sliding window:
 * crates/sapient-models/src/forward/common.rs:355-434 (update_kv_cache, f32
 * cache) and :449-508 (update_kv_cache_q8). cache [n_kv, max_seq, hd] (the
 * reference's [b, h, max_seq, hd] with b·h folded) holds cur_len rows per head.
 * total = cur_len + seq; shift = total − max_seq when positive (:381-383,
 * :465-466): rows [shift, cur_len) of every head move to [0, cur_len − shift),
 * one row at a time in increasing order (copy_within, :392-405 / :475-485),
 * then the new rows are written from insert_pos = cur_len − shift (:408-412,
 * :488-492) — each new row converted as sor_kv_append converts it (Q8_0: the
 * block quantizer of :336-348). Returns the length of the view the reference
 * returns, min(total, max_seq) (:430-433, :510-512), through *new_len.
 * seq > max_seq is the reference's bail (:378-379, :462-463): SOR_ERANGE;
 * cur_len > max_seq, where its subtraction would underflow, SOR_EINVAL. */
int sor_kv_cache_update(const float* src, void* cache, int cache_dtype, size_t n_kv, size_t seq, size_t hd,
                        size_t max_seq, size_t cur_len, size_t* new_len) {
    if (seq > max_seq) return SOR_ERANGE;
    if (cur_len > max_seq) return SOR_EINVAL;
    size_t row_bytes;
    if (cache_dtype == SOR_Q8_0) {
        if (hd % QK != 0) return SOR_EINVAL;
        row_bytes = hd / QK * Q8_0_BYTES;
    } else if (cache_dtype == SOR_F32) {
        row_bytes = hd * 4;
    } else if (cache_dtype == SOR_F16 || cache_dtype == SOR_BF16) {
        row_bytes = hd * 2;
    } else {
        return SOR_EINVAL;
    }
    const size_t total = cur_len + seq;
    const size_t shift = total > max_seq ? total - max_seq : 0;
    if (shift > 0) {
        const size_t keep = cur_len - shift;
        for (size_t h = 0; h < n_kv; h++)
            for (size_t si = 0; si < keep; si++) {
                uint8_t* head = (uint8_t*)cache + h * max_seq * row_bytes;
                memmove(head + si * row_bytes, head + (si + shift) * row_bytes, row_bytes);
            }
    }
    const size_t insert_pos = cur_len - shift;
    const int st = sor_kv_append(src, cache, cache_dtype, n_kv, seq, hd, max_seq, insert_pos);
    if (st != SOR_OK) return st;
    *new_len = total < max_seq ? total : max_seq;
    return SOR_OK;
}
