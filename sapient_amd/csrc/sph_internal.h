// sph_internal.h — entry points shared between the library's translation units
// that are not part of the exported C ABI (hidden symbols).
#pragma once

#include <stdint.h>

extern "C" {

// sph_rope_kv_append with the angles supplied: angles[2 (s·head_dim/2 + i)]
// and [... + 1] hold cos and sin of positions[s] / base^(2i/head_dim), evaluated
// by the caller with the libm the reference calls (rope.hip). Used by the
// decode engine, which knows a step's position on the host.
__attribute__((visibility("hidden"))) int sph_rope_kv_append_angles(
    void* q, int64_t n_q_heads, const void* k, const void* v, int64_t n_kv_heads, int dtype, int layout,
    const int32_t* positions, const float* angles, int64_t seq, int64_t head_dim, void* kcache, void* vcache,
    int cache_dtype, int64_t max_seq, const void* bq, const void* bk, const void* bv, int bias_dtype,
    int32_t* bad_pos_flag, void* stream);

// sph_rope_kv_append_tokens with the angles read from a per-position table:
// angles[2 (p·head_dim/2 + i)] and [... + 1] hold cos and sin of p / base^(2i/head_dim)
// for every position p in [0, max_seq). Token s reads row positions[s], so a
// captured launch serves any positions. Used by the decode engine's chunks.
__attribute__((visibility("hidden"))) int sph_rope_kv_append_tokens_angles(
    const void* q, void* q_out, int64_t n_q_heads, const void* k, const void* v, int64_t n_kv_heads, int dtype,
    int layout, const int32_t* positions, const float* angles, int64_t seq, int64_t head_dim, void* kcache,
    void* vcache, int cache_dtype, int64_t max_seq, const void* bq, const void* bk, const void* bv, int bias_dtype,
    int32_t* bad_pos_flag, void* stream);

}  // extern "C"
