// hip_forward_engine.cpp — the device-resident decode engine of
// sapient_hip_engine.h: sapient's WgpuForwardEngine sequence
// (crates/sapient-models/src/forward/wgpu_engine.rs:362-629) on one HIP stream,
// built from the op set's C ABI.
//
// Differences from the reference's op-by-op sequence, each result-preserving:
//  - `x = add(x, o); h = rms_norm(x)` pairs run as one sph_add_rms_norm
//    (IEEE addition commutes, so o + x is x + o bit for bit);
//  - `add_bias(q|k|v); rope(q); rope(k); kv_append(k); kv_append(v)` runs as
//    one sph_rope_kv_append, bit-exact with that sequence; for a chunk the
//    three transpose_heads before it fold into the same launch
//    (sph_rope_kv_append_tokens reads the projections' token-major rows);
//  - forward_chunk adds the last layer's residual and normalises only the last
//    row, the one the reference slices out before its final norm (:623-627).
//  - RoPE angles, cos and sin of position / base^(2i/hd), are evaluated on the
//    host with the libm the reference calls (the values its own rope
//    computes), so the fused RoPE + KV launch reads them instead of evaluating
//    sin/cos: a one-token step stages its position's angles with the token id
//    and position; a chunk reads rows of a per-position table, the reference's
//    rope_cos_sin_cache (crates/sapient-backends/cpu/src/kernels/rope.rs:140-153)
//    with (cos, sin) interleaved, filled as positions are first reached.
// Decode steps can be captured into a HIP graph once and replayed: every
// per-token value (token id, position, angles) lives in device memory,
// refreshed by one H2D copy from pinned staging before each launch. Chunks
// launch eagerly: a 512-token chunk keeps the GPU busy longer than the host
// takes to issue it, and replaying it from a graph measured slower (611.8
// against 561.3 µs at Qwen2.5-0.5B shape, the op-set part).
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <utility>
#include <vector>

#include "sapient_hip_engine.h"
#include "sph_internal.h"

struct sph_engine {
    sph_engine_config cfg{};
    const void* embed = nullptr;
    int embed_dtype = SPH_F32;
    int64_t vocab = 0;
    std::vector<sph_engine_layer> layers;
    const void* final_norm = nullptr;
    sph_project_fn project = nullptr;
    sph_attend_fn attend = nullptr;
    void* user = nullptr;

    hipStream_t stream = nullptr;
    std::vector<std::pair<void*, size_t>> device_allocs;
    float *x = nullptr, *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *qt = nullptr, *attn = nullptr,
          *attn_sm = nullptr, *o = nullptr, *gate = nullptr, *up = nullptr, *act = nullptr, *down = nullptr,
          *out = nullptr;
    // Per-call inputs of T tokens, packed from byte 0: ids[T], positions[T],
    // then (T = 1) the step's angles, head_dim/2 (cos, sin) pairs. A device
    // buffer and its pinned host staging copy, moved by one H2D copy.
    uint8_t* inputs = nullptr;
    int32_t* flags = nullptr;  // [0] bad token id, [1] bad cache position (both checked on the host first)
    std::vector<void*> kcache, vcache;
    std::vector<float> dens;  // base^(2i/head_dim), i < head_dim/2, from the host libm
    // Row r (< max_seq): head_dim/2 (cos, sin) pairs of position r's angles;
    // rows [0, angle_rows) are filled.
    float* angles = nullptr;
    int64_t angle_rows = 0;

    uint8_t* staged = nullptr;  // pinned
    hipEvent_t staged_done = nullptr;  // the last H2D copy out of the staging buffer
    bool staged_pending = false;

    int64_t cur = 0;
    bool use_graph = false;
    hipGraphExec_t graph = nullptr;  // one-token step
};

namespace {

size_t elem_size(int dt) { return dt == SPH_F32 ? 4 : 2; }

bool is_float(int dt) { return dt == SPH_F32 || dt == SPH_F16 || dt == SPH_BF16; }

void release(sph_engine* e) {
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    if (e->graph) (void)hipGraphExecDestroy(e->graph);
    for (auto& a : e->device_allocs) (void)hipFree(a.first);
    if (e->staged) (void)hipHostFree(e->staged);
    if (e->staged_done) (void)hipEventDestroy(e->staged_done);
    if (e->stream) (void)hipStreamDestroy(e->stream);
}

template <typename T>
bool dalloc(sph_engine* e, T** p, size_t bytes) {
    void* ptr = nullptr;
    if (bytes == 0) bytes = 16;
    if (hipMalloc(&ptr, bytes) != hipSuccess) return false;
    e->device_allocs.emplace_back(ptr, bytes);
    *p = static_cast<T*>(ptr);
    return true;
}

// Host-side view of a callback's status: 0 is success, an SPH_* code passes
// through, anything else reads as a HIP failure.
int callback_status(int st) {
    if (st == 0) return SPH_OK;
    return (st == SPH_EINVAL || st == SPH_EHIP || st == SPH_ERANGE || st == SPH_ENODEV || st == SPH_ESTATE) ? st : SPH_EHIP;
}

int proj(sph_engine* e, int layer, int which, const float* in, float* out, int64_t rows) {
    if (!e->project) return SPH_OK;
    return callback_status(e->project(e->user, layer, which, in, out, rows, e->stream));
}

#define SPH_TRY(expr)                \
    do {                             \
        const int st_ = (expr);      \
        if (st_ != SPH_OK) return st_; \
    } while (0)

const uint32_t* ids_of(const sph_engine* e) { return reinterpret_cast<const uint32_t*>(e->inputs); }
int32_t* positions_of(const sph_engine* e, int64_t T) { return reinterpret_cast<int32_t*>(e->inputs + 4 * T); }
const float* angles_of(const sph_engine* e) { return reinterpret_cast<const float*>(e->inputs + 8); }  // T = 1

// Everything one forward call enqueues after its inputs are staged: T tokens
// whose ids and positions (and, for one token, angles) are in device memory.
int body(sph_engine* e, int64_t T) {
    const sph_engine_config& c = e->cfg;
    hipStream_t s = e->stream;
    int32_t* positions = positions_of(e, T);
    SPH_TRY(sph_embed(e->embed, e->embed_dtype, e->vocab, c.hidden, ids_of(e), T, e->x, e->flags, s));
    for (int l = 0; l < (int)c.n_layers; ++l) {
        const sph_engine_layer& L = e->layers[l];
        // attention block: h = rms_norm(x) (layer 0) or x += down; h = rms_norm(x)
        if (l == 0)
            SPH_TRY(sph_rms_norm(e->x, SPH_F32, L.input_ln, SPH_F32, e->h, SPH_F32, T, c.hidden, c.rms_eps, s));
        else
            SPH_TRY(sph_add_rms_norm(e->down, e->x, SPH_F32, L.input_ln, SPH_F32, e->h, SPH_F32, T, c.hidden,
                                     c.rms_eps, s));
        SPH_TRY(proj(e, l, SPH_PROJ_Q, e->h, e->q, T));
        SPH_TRY(proj(e, l, SPH_PROJ_K, e->h, e->k, T));
        SPH_TRY(proj(e, l, SPH_PROJ_V, e->h, e->v, T));
        // q/k/v biases, RoPE and the cache append in one launch. One token: token-major
        // [1, heads, hd] is heads-major already, q is rotated in place. A chunk: q, k, v
        // are read token-major and q is written heads-major to qt, the transposes fused.
        float* qh = e->q;
        if (T == 1) {
            SPH_TRY(sph_rope_kv_append_angles(e->q, c.n_heads, e->k, e->v, c.n_kv_heads, SPH_F32, c.rope_layout,
                                              positions, angles_of(e), T, c.head_dim, e->kcache[l], e->vcache[l],
                                              c.kv_dtype, c.max_seq, L.bq, L.bk, L.bv, c.bias_dtype, e->flags + 1,
                                              s));
        } else {
            // Each token reads the angle-table row its position names.
            qh = e->qt;
            SPH_TRY(sph_rope_kv_append_tokens_angles(e->q, e->qt, c.n_heads, e->k, e->v, c.n_kv_heads, SPH_F32,
                                                     c.rope_layout, positions, e->angles, T, c.head_dim,
                                                     e->kcache[l], e->vcache[l], c.kv_dtype, c.max_seq, L.bq, L.bk,
                                                     L.bv, c.bias_dtype, e->flags + 1, s));
        }
        if (e->attend)
            SPH_TRY(callback_status(e->attend(e->user, l, qh, e->kcache[l], e->vcache[l], c.kv_dtype, positions, T,
                                              c.max_seq, e->attn, s)));
        float* att = e->attn;
        if (T > 1) {
            SPH_TRY(sph_transpose_heads(e->attn, e->attn_sm, SPH_F32, c.n_heads, T, c.head_dim, s));
            att = e->attn_sm;
        }
        SPH_TRY(proj(e, l, SPH_PROJ_O, att, e->o, T));
        if (L.bo) SPH_TRY(sph_add_bias(e->o, L.bo, c.bias_dtype, e->o, SPH_F32, T * c.hidden, c.hidden, s));
        // MLP block: x += o; h = rms_norm(x); act = swiglu(gate(h), up(h)); down(act)
        SPH_TRY(sph_add_rms_norm(e->o, e->x, SPH_F32, L.post_ln, SPH_F32, e->h, SPH_F32, T, c.hidden, c.rms_eps, s));
        SPH_TRY(proj(e, l, SPH_PROJ_GATE, e->h, e->gate, T));
        SPH_TRY(proj(e, l, SPH_PROJ_UP, e->h, e->up, T));
        SPH_TRY(sph_swiglu(e->gate, e->up, e->act, SPH_F32, T * c.intermediate, s));
        SPH_TRY(proj(e, l, SPH_PROJ_DOWN, e->act, e->down, T));
    }
    // x += down and the final norm, for the last token only.
    const size_t last = (size_t)(T - 1) * (size_t)c.hidden;
    return sph_add_rms_norm(e->down + last, e->x + last, SPH_F32, e->final_norm, SPH_F32, e->out, SPH_F32, 1,
                            c.hidden, c.rms_eps, s);
}

// The reference's angle: freq = (f32)pos / base^(2i/d), then cosf / sinf
// (rope.rs:48-57); pos_scale 1 divides exactly. Writes (cos, sin) pairs.
void angles_at(const sph_engine* e, int64_t pos, float* out) {
    const float p = (float)pos;
    for (size_t i = 0; i < e->dens.size(); ++i) {
        const float freq = p / e->dens[i];
        out[2 * i] = cosf(freq);
        out[2 * i + 1] = sinf(freq);
    }
}

// Fill the angle table up to row `need` (<= max_seq). It grows by doubling,
// at least 256 rows at a time, so a run of chunks uploads O(log max_seq)
// times; each upload completes before the call returns, and rows already on
// the device are never rewritten.
int fill_angles(sph_engine* e, int64_t need) {
    if (need <= e->angle_rows) return SPH_OK;
    const int64_t rows = std::min(e->cfg.max_seq, std::max({need, 2 * e->angle_rows, (int64_t)256}));
    const size_t row = (size_t)e->cfg.head_dim;  // floats per row
    try {
        std::vector<float> buf((size_t)(rows - e->angle_rows) * row);
        for (int64_t r = e->angle_rows; r < rows; ++r) angles_at(e, r, buf.data() + (size_t)(r - e->angle_rows) * row);
        if (hipMemcpyAsync(e->angles + (size_t)e->angle_rows * row, buf.data(), buf.size() * 4,
                           hipMemcpyHostToDevice, e->stream) != hipSuccess ||
            hipStreamSynchronize(e->stream) != hipSuccess)
            return SPH_EHIP;
    } catch (...) {
        return SPH_EHIP;
    }
    e->angle_rows = rows;
    return SPH_OK;
}

// Copy ids and positions cur .. cur + n - 1 to the device (checked first).
int stage(sph_engine* e, const uint32_t* toks, int64_t n) {
    if (n <= 0 || n > e->cfg.max_chunk) return SPH_EINVAL;
    if (e->cur + n > e->cfg.max_seq) return SPH_ERANGE;
    for (int64_t i = 0; i < n; ++i)
        if ((int64_t)toks[i] >= e->vocab) return SPH_ERANGE;
    if (e->staged_pending && hipEventSynchronize(e->staged_done) != hipSuccess) return SPH_EHIP;
    std::memcpy(e->staged, toks, (size_t)n * 4);
    int32_t* pos = reinterpret_cast<int32_t*>(e->staged + 4 * n);
    for (int64_t i = 0; i < n; ++i) pos[i] = (int32_t)(e->cur + i);
    size_t bytes = (size_t)n * 8;
    if (n == 1) {
        angles_at(e, e->cur, reinterpret_cast<float*>(e->staged + 8));
        bytes += e->dens.size() * 8;
    }
    if (hipMemcpyAsync(e->inputs, e->staged, bytes, hipMemcpyHostToDevice, e->stream) != hipSuccess ||
        hipEventRecord(e->staged_done, e->stream) != hipSuccess)
        return SPH_EHIP;
    e->staged_pending = true;
    return SPH_OK;
}

int capture_decode(sph_engine* e) {
    if (hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) return SPH_EHIP;
    const int st = body(e, 1);
    hipGraph_t g = nullptr;
    const hipError_t end = hipStreamEndCapture(e->stream, &g);
    if (st != SPH_OK || end != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return st != SPH_OK ? st : SPH_EHIP;
    }
    const hipError_t inst = hipGraphInstantiate(&e->graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (inst != hipSuccess) {
        e->graph = nullptr;
        return SPH_EHIP;
    }
    return SPH_OK;
}

}  // namespace

extern "C" int sph_engine_create(const sph_engine_config* cfg, const void* embed_table, int embed_dtype,
                                 int64_t vocab, const sph_engine_layer* layers, const void* final_norm,
                                 sph_project_fn project, sph_attend_fn attend, void* user, sph_engine** out) {
    if (!cfg || !embed_table || !layers || !final_norm || !out) return SPH_EINVAL;
    *out = nullptr;
    const sph_engine_config& c = *cfg;
    if (c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 || c.intermediate <= 0 ||
        c.n_layers <= 0 || c.max_seq <= 0 || c.max_chunk <= 0 || vocab <= 0)
        return SPH_EINVAL;
    if (c.n_heads % c.n_kv_heads != 0 || c.head_dim % 2 != 0 || c.max_seq > INT32_MAX) return SPH_EINVAL;
    if (c.rope_layout != SPH_ROPE_NEOX && c.rope_layout != SPH_ROPE_INTERLEAVED) return SPH_EINVAL;
    if (!is_float(c.kv_dtype) || !is_float(c.bias_dtype)) return SPH_EINVAL;
    for (int64_t l = 0; l < c.n_layers; ++l)
        if (!layers[l].input_ln || !layers[l].post_ln) return SPH_EINVAL;

    sph_engine* e = new (std::nothrow) sph_engine;
    if (!e) return SPH_EINVAL;
    // The host-side vectors below may throw std::bad_alloc; nothing may unwind
    // through the C ABI, so a failed allocation of any kind returns SPH_EHIP.
    bool ok = false;
    try {
        e->cfg = c;
        e->dens.resize((size_t)(c.head_dim / 2));
        for (size_t i = 0; i < e->dens.size(); ++i)
            e->dens[i] = powf(c.rope_theta, 2.0f * (float)i / (float)c.head_dim);
        e->embed = embed_table;
        e->embed_dtype = embed_dtype;
        e->vocab = vocab;
        e->layers.assign(layers, layers + c.n_layers);
        e->final_norm = final_norm;
        e->project = project;
        e->attend = attend;
        e->user = user;

        const size_t T = (size_t)c.max_chunk;
        const size_t qd = (size_t)(c.n_heads * c.head_dim), kd = (size_t)(c.n_kv_heads * c.head_dim);
        const size_t cache_bytes =
            (size_t)c.n_kv_heads * (size_t)c.max_seq * (size_t)c.head_dim * elem_size(c.kv_dtype);
        ok = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) == hipSuccess &&
                  hipEventCreateWithFlags(&e->staged_done, hipEventDisableTiming) == hipSuccess &&
                  hipHostMalloc((void**)&e->staged, T * 8 + (size_t)c.head_dim * 4, hipHostMallocDefault) ==
                      hipSuccess &&
                  dalloc(e, &e->x, T * c.hidden * 4) && dalloc(e, &e->h, T * c.hidden * 4) &&
                  dalloc(e, &e->q, T * qd * 4) &&
                  dalloc(e, &e->k, T * kd * 4) && dalloc(e, &e->v, T * kd * 4) && dalloc(e, &e->qt, T * qd * 4) &&
                  dalloc(e, &e->attn, T * qd * 4) &&
                  dalloc(e, &e->attn_sm, T * qd * 4) && dalloc(e, &e->o, T * c.hidden * 4) &&
                  dalloc(e, &e->gate, T * c.intermediate * 4) && dalloc(e, &e->up, T * c.intermediate * 4) &&
                  dalloc(e, &e->act, T * c.intermediate * 4) && dalloc(e, &e->down, T * c.hidden * 4) &&
                  dalloc(e, &e->out, (size_t)c.hidden * 4) && dalloc(e, &e->inputs, T * 8 + (size_t)c.head_dim * 4) &&
                  dalloc(e, &e->flags, 2 * 4) && dalloc(e, &e->angles, (size_t)c.max_seq * (size_t)c.head_dim * 4);
        for (int64_t l = 0; ok && l < c.n_layers; ++l) {
            void *kc = nullptr, *vc = nullptr;
            ok = dalloc(e, &kc, cache_bytes) && dalloc(e, &vc, cache_bytes);
            e->kcache.push_back(kc);
            e->vcache.push_back(vc);
        }
        // Buffers a NULL callback leaves untouched start at zero, as do the caches.
        for (size_t i = 0; ok && i < e->device_allocs.size(); ++i)
            ok = hipMemsetAsync(e->device_allocs[i].first, 0, e->device_allocs[i].second, e->stream) == hipSuccess;
        ok = ok && hipStreamSynchronize(e->stream) == hipSuccess;
    } catch (...) {
        ok = false;
    }
    if (!ok) {
        release(e);
        delete e;
        return SPH_EHIP;
    }
    *out = e;
    return SPH_OK;
}

extern "C" void sph_engine_destroy(sph_engine* e) {
    if (!e) return;
    release(e);
    delete e;
}

extern "C" int sph_engine_forward_token(sph_engine* e, uint32_t tok, const float** hidden) {
    if (!e || !hidden) return SPH_EINVAL;
    SPH_TRY(stage(e, &tok, 1));
    if (e->use_graph) {
        if (!e->graph) SPH_TRY(capture_decode(e));
        if (hipGraphLaunch(e->graph, e->stream) != hipSuccess) return SPH_EHIP;
    } else {
        SPH_TRY(body(e, 1));
    }
    e->cur += 1;
    *hidden = e->out;
    return SPH_OK;
}

extern "C" int sph_engine_forward_chunk(sph_engine* e, const uint32_t* toks, int64_t n, const float** hidden) {
    if (!e || !toks || !hidden) return SPH_EINVAL;
    SPH_TRY(stage(e, toks, n));
    if (n > 1) SPH_TRY(fill_angles(e, e->cur + n));
    SPH_TRY(body(e, n));
    e->cur += n;
    *hidden = e->out;
    return SPH_OK;
}

extern "C" int sph_engine_use_graph(sph_engine* e, int on) {
    if (!e) return SPH_EINVAL;
    e->use_graph = on != 0;
    return SPH_OK;
}

extern "C" int sph_engine_reset(sph_engine* e) {
    if (!e) return SPH_EINVAL;
    e->cur = 0;
    return SPH_OK;
}

extern "C" int64_t sph_engine_position(const sph_engine* e) { return e ? e->cur : -1; }
extern "C" void* sph_engine_stream(const sph_engine* e) { return e ? (void*)e->stream : nullptr; }
extern "C" const void* sph_engine_kcache(const sph_engine* e, int layer) {
    return e && layer >= 0 && layer < (int)e->kcache.size() ? e->kcache[layer] : nullptr;
}
extern "C" const void* sph_engine_vcache(const sph_engine* e, int layer) {
    return e && layer >= 0 && layer < (int)e->vcache.size() ? e->vcache[layer] : nullptr;
}
