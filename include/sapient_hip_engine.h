/*
 * sapient_hip_engine.h — a device-resident decode engine over the op set of
 * sapient_hip.h, for callers that keep a model's activations on one MI355X.
 *
 * It is the HIP counterpart of sapient's WgpuForwardEngine
 * (crates/sapient-models/src/forward/wgpu_engine.rs:362-629): the same per-layer
 * sequence for a Llama-family decoder — embed → per layer {RMSNorm → Q/K/V
 * projections (+bias) → RoPE → KV-cache append → attention → O projection
 * (+bias) → residual add → RMSNorm → gate/up projections → SwiGLU → down
 * projection → residual add} → final RMSNorm — with every residual add fused
 * into the RMSNorm that follows it and RoPE fused with the cache append.
 * Projections and attention are outside this library: the caller supplies them
 * as callbacks that enqueue their own work on the engine's stream.
 *
 * Activations are f32 (as the wgpu engine's); the KV cache is F32, F16 or BF16.
 * All device memory is allocated by sph_engine_create; the forward calls
 * allocate nothing. With sph_engine_use_graph(e, 1) the first decode step is
 * captured into a HIP graph and later steps replay it: the token id and
 * position are copied to device memory before each launch, so callbacks must
 * read the position from the `positions` pointer they are given (not bake it)
 * and must be capturable (no allocation, no synchronization, no
 * hipMemsetAsync).
 *
 * Status codes are those of sapient_hip.h; SPH_ERANGE reports a full KV cache
 * or a token id ≥ vocab, before any work is enqueued.
 */
#ifndef SAPIENT_HIP_ENGINE_H
#define SAPIENT_HIP_ENGINE_H

#include <stdint.h>

#include "sapient_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sph_engine sph_engine;

typedef struct {
    int64_t hidden, n_heads, n_kv_heads, head_dim, intermediate, n_layers;
    int64_t max_seq;   /* KV-cache positions */
    int64_t max_chunk; /* most tokens one sph_engine_forward_chunk may take */
    float rms_eps, rope_theta;
    int rope_layout; /* SPH_ROPE_NEOX or SPH_ROPE_INTERLEAVED; rotary_dim = head_dim */
    int kv_dtype;    /* SPH_F32, SPH_F16 or SPH_BF16 */
    int bias_dtype;  /* element type of the biases: SPH_F32, SPH_F16 or SPH_BF16 (norm weights are f32) */
} sph_engine_config;

/* Device pointers of one layer's weights handled here; biases may be NULL. */
typedef struct {
    const void* input_ln; /* [hidden] f32 */
    const void* post_ln;  /* [hidden] f32 */
    const void* bq;       /* [n_heads · head_dim] */
    const void* bk;       /* [n_kv_heads · head_dim] */
    const void* bv;       /* [n_kv_heads · head_dim] */
    const void* bo;       /* [hidden] */
} sph_engine_layer;

enum { SPH_PROJ_Q = 0, SPH_PROJ_K = 1, SPH_PROJ_V = 2, SPH_PROJ_O = 3, SPH_PROJ_GATE = 4, SPH_PROJ_UP = 5,
       SPH_PROJ_DOWN = 6 };

/* out[rows, n_out] = in[rows, n_in] · W^T for projection `which` of `layer`
 * (n_in / n_out implied by the config); rows-major f32. Enqueue on `stream`
 * and return 0, or a nonzero status that aborts the forward call. */
typedef int (*sph_project_fn)(void* user, int layer, int which, const float* in, float* out, int64_t rows,
                              void* stream);

/* Causal attention of n_tok queries q [n_heads, n_tok, head_dim] (heads-major,
 * rotated) over cache rows 0 .. positions[t] of kcache / vcache [n_kv_heads,
 * max_seq, head_dim] (kv_dtype) into out [n_heads, n_tok, head_dim] f32.
 * positions is device int32[n_tok]. */
typedef int (*sph_attend_fn)(void* user, int layer, const float* q, const void* kcache, const void* vcache,
                             int kv_dtype, const int32_t* positions, int64_t n_tok, int64_t max_seq, float* out,
                             void* stream);

/* `embed_table`: raw table bytes ([vocab, hidden] of embed_dtype, as sph_embed);
 * `layers`: n_layers entries; `final_norm`: [hidden] f32. A NULL callback skips its
 * stage (the output buffer keeps its contents) — for timing this library's part. */
int sph_engine_create(const sph_engine_config* cfg, const void* embed_table, int embed_dtype, int64_t vocab,
                      const sph_engine_layer* layers, const void* final_norm, sph_project_fn project,
                      sph_attend_fn attend, void* user, sph_engine** out);
void sph_engine_destroy(sph_engine* e);

/* One token at the next position (WgpuForwardEngine::forward_token). On
 * success *hidden = the device f32 [hidden] final hidden state, valid until the
 * next call; the work is enqueued on the engine's stream, not waited for. */
int sph_engine_forward_token(sph_engine* e, uint32_t tok, const float** hidden);
/* n ≤ max_chunk tokens at the next positions (WgpuForwardEngine::forward_chunk);
 * *hidden = the final hidden state of the last token. The first chunk to reach
 * a position beyond the engine's RoPE angle table extends it from the host
 * and waits for that upload (and so for the stream's earlier work); the table
 * grows by doubling, so this happens O(log max_seq) times. */
int sph_engine_forward_chunk(sph_engine* e, const uint32_t* toks, int64_t n, const float** hidden);
/* Replay forward_token from a captured HIP graph (1) or launch eagerly (0);
 * forward_chunk always launches eagerly. */
int sph_engine_use_graph(sph_engine* e, int on);
/* Start again at position 0 (cached rows are overwritten as positions refill). */
int sph_engine_reset(sph_engine* e);
int64_t sph_engine_position(const sph_engine* e);
void* sph_engine_stream(const sph_engine* e);
const void* sph_engine_kcache(const sph_engine* e, int layer);
const void* sph_engine_vcache(const sph_engine* e, int layer);

#ifdef __cplusplus
}
#endif

#endif /* SAPIENT_HIP_ENGINE_H */
