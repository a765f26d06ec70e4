// GPU tests of the C++ LlmBackend mirror (include/sapient_hip_backend.hpp),
// written after the reference's own unit tests so they read the same way:
//   layernorm.rs:113-149, elementwise.rs:176-232, rope.rs:155-206,
//   common.rs:556-569 and :669-718, the KV-cache update (tests/inference_test.rs:10-61 and the
//   sliding window of common.rs:355-528), the graph-side dispatch arms of
//   crates/sapient-backends/cpu/src/backend.rs:239-487, the trait's validation errors (rope.rs:19-35,
//   elementwise.rs:15-21, common.rs:171-173), and the debug switches of backend.rs:191-216.
// Prints "test <name> ... ok|FAILED: <why>" per test; exits 1 if any failed.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include <hip/hip_runtime.h>

#include "sapient_hip_backend.hpp"

using sapient_hip::Bytes;
using sapient_hip::byte_count;
using sapient_hip::DType;
using sapient_hip::Error;
using sapient_hip::HipLlmBackend;
using sapient_hip::Tensor;

struct Failure {
    std::string why;
};

#define ASSERT(cond, msg) \
    do {                  \
        if (!(cond)) throw Failure{std::string(msg) + " [" #cond "]"}; \
    } while (0)

template <typename F>
static std::string expect_error(F&& f) {
    try {
        f();
    } catch (const Error& e) {
        return e.what();
    }
    throw Failure{"expected an error"};
}

static bool same_bytes(const Bytes& a, const std::vector<uint8_t>& b) {
    return a.size() == b.size() && std::equal(a.begin(), a.end(), b.begin());
}

// ── helpers the reference tests use ──────────────────────────────────────────
static uint16_t f16_from_f32(float f) {  // half::f16::from_f32 (nearest-even)
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xFFu, man = x & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0u));
    const int e = (int)exp - 112;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        const uint32_t m = man | 0x800000u, sh = (uint32_t)(14 - e);
        uint32_t h = m >> sh;
        const uint32_t rb = 1u << (sh - 1);
        if ((m & rb) && ((m & (rb - 1)) || (h & 1))) ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    if ((man & 0x1000u) && (man & 0x2FFFu)) ++h;
    return (uint16_t)h;
}

static float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    uint32_t u;
    if (exp == 0x1F) u = sign | 0x7F800000u | (man << 13);
    else if (exp == 0) {
        float f = (float)man * 0x1p-24f;
        std::memcpy(&u, &f, 4);
        u |= sign;
    } else u = sign | ((exp + 112u) << 23) | (man << 13);
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// quantize_q8_0_block (crates/sapient-backends/cpu/src/kernels/quant.rs:223-235)
static std::vector<uint8_t> quantize_q8_0(const std::vector<float>& x) {
    std::vector<uint8_t> out;
    for (size_t b = 0; b < x.size() / 32; ++b) {
        float max_abs = 0.0f;
        for (int i = 0; i < 32; ++i) max_abs = std::fmax(max_abs, std::fabs(x[b * 32 + i]));
        const float scale = max_abs / 127.0f;
        const uint16_t d = f16_from_f32(scale);
        const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        out.push_back((uint8_t)(d & 0xFF));
        out.push_back((uint8_t)(d >> 8));
        for (int i = 0; i < 32; ++i) {
            float q = std::round(x[b * 32 + i] * inv);
            q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
            out.push_back((uint8_t)(int8_t)q);
        }
    }
    return out;
}

// ── tests ────────────────────────────────────────────────────────────────────
static void rmsnorm_identity_weight(HipLlmBackend& bk) {  // layernorm.rs:125-149
    const Tensor x = Tensor::from_f32({3.0f, 4.0f}, {1, 2});
    const Tensor w = Tensor::from_f32({1.0f, 1.0f}, {2});
    const std::vector<float> d = bk.rms_norm(x, w, 0.0f).as_f32();
    const float e0 = 3.0f / std::sqrt(12.5f), e1 = 4.0f / std::sqrt(12.5f);
    ASSERT(std::fabs(d[0] - e0) < 1e-5f && std::fabs(d[1] - e1) < 1e-5f, "rms_norm [3,4]");
}

static void rmsnorm_half_input_outputs_f32(HipLlmBackend& bk) {  // to_f32_cow upcast, f32 result
    Bytes b;
    for (float v : {3.0f, 4.0f}) {
        const uint16_t h = f16_from_f32(v);
        b.push_back((uint8_t)(h & 0xFF));
        b.push_back((uint8_t)(h >> 8));
    }
    const Tensor y = bk.rms_norm(Tensor::from_f16_bytes(b, {1, 2}), Tensor::from_f32({1.0f, 1.0f}, {2}), 0.0f);
    ASSERT(y.dtype() == DType::F32, "f32 output");
    ASSERT(std::fabs(y.as_f32()[1] - 4.0f / std::sqrt(12.5f)) < 1e-5f, "value");
}

static void layernorm_zero_mean_unit_var(HipLlmBackend& bk) {  // layernorm.rs:113-123 (unit weight)
    const Tensor x = Tensor::from_f32({1.0f, 2.0f, 3.0f, 4.0f}, {2, 2});
    const std::vector<float> d = bk.layer_norm(x, Tensor::from_f32({1.0f, 1.0f}, {2}), nullptr, 1e-5f).as_f32();
    ASSERT(std::fabs(d[0] + 1.0f) < 1e-4f && std::fabs(d[1] - 1.0f) < 1e-4f, "row 0");
    ASSERT(std::fabs(d[2] + 1.0f) < 1e-4f && std::fabs(d[3] - 1.0f) < 1e-4f, "row 1");
    const Tensor b = Tensor::from_f32({0.5f, -0.5f}, {2});
    const std::vector<float> e = bk.layer_norm(x, Tensor::from_f32({2.0f, 2.0f}, {2}), &b, 1e-5f).as_f32();
    ASSERT(std::fabs(e[0] + 1.5f) < 2e-4f && std::fabs(e[1] - 1.5f) < 2e-4f, "weight and bias");
    ASSERT(expect_error([&] { bk.layer_norm(x, Tensor::from_f32({1.0f}, {1}), nullptr, 1e-5f); })
               .find("shape mismatch") != std::string::npos, "weight length");
}

static void test_gelu_erf(HipLlmBackend& bk) {  // elementwise.rs:216-224
    const std::vector<float> v = bk.gelu_erf(Tensor::from_f32({0.0f, 1.0f, -1.0f}, {3})).as_f32();
    ASSERT(std::fabs(v[0]) < 1e-6f, "g(0)");
    ASSERT(std::fabs(v[1] - 0.8413447f) < 1e-4f, "g(1)");
    ASSERT(std::fabs(v[2] + 0.1586553f) < 1e-4f, "g(-1)");
}

static void add_bias_last_dim_broadcasts(HipLlmBackend& bk) {  // common.rs:556-569
    const Tensor y = Tensor::from_f32({1.0f, 2.0f, 3.0f, 4.0f, 5.0f, 6.0f}, {2, 3});
    const std::vector<float> o = bk.add_bias_last_dim(y, Tensor::from_f32({10.0f, 20.0f, 30.0f}, {3})).as_f32();
    ASSERT(o == std::vector<float>({11.0f, 22.0f, 33.0f, 14.0f, 25.0f, 36.0f}), "f32 bias");
    Bytes hb;
    for (float v : {0.5f, -1.0f, 2.0f}) {
        const uint16_t h = f16_from_f32(v);
        hb.push_back((uint8_t)(h & 0xFF));
        hb.push_back((uint8_t)(h >> 8));
    }
    const std::vector<float> h = bk.add_bias_last_dim(y, Tensor::from_f16_bytes(hb, {3})).as_f32();
    ASSERT(h == std::vector<float>({1.5f, 1.0f, 5.0f, 4.5f, 4.0f, 8.0f}), "f16 bias");
    const std::string e = expect_error([&] { bk.add_bias_last_dim(y, Tensor::from_f32({1.0f, 2.0f}, {2})); });
    ASSERT(e.find("bias length 2 does not match last dim 3") != std::string::npos, "length error");
}

// ── graph-side dispatch (cpu/src/backend.rs:239-487) ──────────────────────────
static void graph_rms_norm_optional_weight(HipLlmBackend& bk) {  // :313-320 with inputs.get(1) = None
    sapient_hip::HipExecutionBackend ex(bk);
    const Tensor x = Tensor::from_f32({3.0f, 4.0f}, {1, 2});
    sapient_hip::OpAttrs a;
    a.epsilon = 0.0f;
    const std::vector<float> d = ex.dispatch(sapient_hip::OpKind::RmsNorm, a, {&x}).at(0).as_f32();
    ASSERT(std::fabs(d[0] - 3.0f / std::sqrt(12.5f)) < 1e-5f && std::fabs(d[1] - 4.0f / std::sqrt(12.5f)) < 1e-5f,
           "unit-weight rms_norm");
}

static void graph_layer_norm_axis(HipLlmBackend& bk) {  // :302-312, axis = 1 on [2, 2, 2]
    sapient_hip::HipExecutionBackend ex(bk);
    const std::vector<float> v = {1, 2, 3, 4, 10, 20, 30, 40};
    const Tensor x = Tensor::from_f32(v, {2, 2, 2});
    sapient_hip::OpAttrs a;
    a.axis = 1;
    a.epsilon = 1e-5f;
    const std::vector<float> d = ex.dispatch(sapient_hip::OpKind::LayerNorm, a, {&x}).at(0).as_f32();
    for (int r = 0; r < 2; ++r) {  // each outer row normalises 4 values
        double m = 0, var = 0;
        for (int i = 0; i < 4; ++i) m += v[r * 4 + i] / 4.0;
        for (int i = 0; i < 4; ++i) var += (v[r * 4 + i] - m) * (v[r * 4 + i] - m) / 4.0;
        for (int i = 0; i < 4; ++i)
            ASSERT(std::fabs(d[r * 4 + i] - (v[r * 4 + i] - m) / std::sqrt(var + 1e-5)) < 1e-5, "layer_norm axis 1");
    }
}

static void graph_embedding_ids_and_shape(HipLlmBackend& bk) {  // :381-411
    sapient_hip::HipExecutionBackend ex(bk);
    std::vector<float> table(5 * 4);
    for (size_t i = 0; i < table.size(); ++i) table[i] = (float)i;
    const Tensor w = Tensor::from_f32(table, {5, 4});
    const Tensor ids_f = Tensor::from_f32({4.0f, 0.0f, 2.0f}, {1, 3});  // F32 ids, cast as Rust `as u32`
    const Tensor out = ex.dispatch(sapient_hip::OpKind::Embedding, {}, {&w, &ids_f}).at(0);
    ASSERT(out.shape() == std::vector<size_t>({1, 3, 4}), "output [batch, seq, hidden]");
    const std::vector<float> o = out.as_f32();
    for (int c = 0; c < 4; ++c)
        ASSERT(o[c] == 16.0f + c && o[4 + c] == (float)c && o[8 + c] == 8.0f + c, "gathered rows");
    const std::string e = expect_error([&] {
        const Tensor bad = Tensor::from_f32({5.0f}, {1, 1});
        ex.dispatch(sapient_hip::OpKind::Embedding, {}, {&w, &bad});
    });
    ASSERT(e.find("out of vocab range") != std::string::npos, "id >= vocab");
}

static void graph_rope_positions_from_seq(HipLlmBackend& bk) {  // :480-487: positions 0 .. dims[2]
    sapient_hip::HipExecutionBackend ex(bk);
    std::vector<float> data;
    for (int i = 0; i < 2 * 3 * 8; ++i) data.push_back(0.05f * (float)i - 1.0f);
    const Tensor x = Tensor::from_f32(data, {1, 2, 3, 8});
    sapient_hip::OpAttrs a;
    a.base = 10000.0f;
    const std::vector<float> g = ex.dispatch(sapient_hip::OpKind::RotaryEmbedding, a, {&x}).at(0).as_f32();
    const std::vector<float> w = bk.apply_rope_positions(x, {0, 1, 2}, 10000.0f).as_f32();
    ASSERT(g == w, "graph RoPE == apply_rope_positions(0..S)");
    ASSERT(sapient_hip::HipExecutionBackend::supports_op(sapient_hip::OpKind::RotaryEmbedding), "supports_op");
}

static void test_add(HipLlmBackend& bk) {  // elementwise.rs:184-194
    const std::vector<float> r = bk.add(Tensor::from_f32({1.0f, 2.0f}, {2}), Tensor::from_f32({3.0f, 4.0f}, {2})).as_f32();
    ASSERT(std::fabs(r[0] - 4.0f) < 1e-6f && r[1] == 6.0f, "add");
}

static void test_scalar_broadcast(HipLlmBackend& bk) {  // elementwise.rs:225-231
    const Tensor a = Tensor::from_f32({1.0f, 2.0f, 3.0f}, {3});
    const Tensor b = Tensor::from_f32({2.0f}, {1});
    ASSERT(bk.mul(a, b).as_f32() == std::vector<float>({2.0f, 4.0f, 6.0f}), "mul broadcast b");
    ASSERT(bk.mul(b, a).as_f32() == std::vector<float>({2.0f, 4.0f, 6.0f}), "mul broadcast a");
    const std::string e = expect_error([&] { bk.add(a, Tensor::from_f32({1.0f, 2.0f}, {2})); });
    ASSERT(e.find("shape mismatch") != std::string::npos, "mismatch error");
}

static void test_gelu(HipLlmBackend& bk) {  // elementwise.rs:206-210
    ASSERT(std::fabs(bk.gelu(Tensor::from_f32({0.0f}, {1})).as_f32()[0]) < 1e-5f, "gelu(0)");
}

static void test_silu_and_swiglu(HipLlmBackend& bk) {  // silu(0) = 0, silu(x) = x·sigmoid(x)
    const std::vector<float> s = bk.silu(Tensor::from_f32({0.0f, 1.0f, -2.0f}, {3})).as_f32();
    ASSERT(s[0] == 0.0f, "silu(0)");
    ASSERT(std::fabs(s[1] - 1.0f / (1.0f + std::exp(-1.0f))) < 1e-6f, "silu(1)");
    ASSERT(std::fabs(s[2] + 2.0f / (1.0f + std::exp(2.0f))) < 1e-6f, "silu(-2)");
    const Tensor g = Tensor::from_f32({0.5f, -1.5f, 3.0f}, {3});
    const Tensor u = Tensor::from_f32({2.0f, 0.25f, -1.0f}, {3});
    const std::vector<float> sw = bk.swiglu(g, u).as_f32();
    const std::vector<float> composed = bk.mul(bk.silu(g), u).as_f32();
    ASSERT(sw == composed, "swiglu == mul(silu(g), u) bit for bit");
}

static void unary_rejects_non_f32(HipLlmBackend& bk) {  // elementwise.rs:15-21
    const Tensor h = Tensor::from_f16_bytes({0, 0, 0, 0}, {2});
    ASSERT(expect_error([&] { bk.silu(h); }).find("type mismatch") != std::string::npos, "silu");
    ASSERT(expect_error([&] { bk.gelu(h); }).find("type mismatch") != std::string::npos, "gelu");
}

static void rope_output_shape(HipLlmBackend& bk) {  // rope.rs:159-165
    const Tensor x = Tensor::from_f32(std::vector<float>(64, 0.1f), {1, 2, 4, 8});
    ASSERT(bk.apply_rope_positions(x, {0, 1, 2, 3}, 10000.0f).shape() == std::vector<size_t>({1, 2, 4, 8}), "shape");
}

static void rope_partial_leaves_tail_unchanged(HipLlmBackend& bk) {  // rope.rs:167-181
    std::vector<float> data;
    for (int v = 1; v <= 8; ++v) data.push_back((float)v);
    const std::vector<float> o = bk.apply_rope_partial(Tensor::from_f32(data, {1, 1, 1, 8}), {3}, 10000.0f, 4).as_f32();
    for (int i = 4; i < 8; ++i) ASSERT(std::fabs(o[i] - data[i]) < 1e-6f, "tail channel changed");
    bool any = false;
    for (int i = 0; i < 4; ++i) any |= std::fabs(o[i] - data[i]) > 1e-6f;
    ASSERT(any, "rotary channels changed");
}

static void rope_partial_full_matches_apply_rope(HipLlmBackend& bk) {  // rope.rs:183-193
    std::vector<float> data;
    for (int v = 0; v < 16; ++v) data.push_back((float)v * 0.1f);
    const Tensor x = Tensor::from_f32(data, {1, 1, 2, 8});
    const std::vector<float> full = bk.apply_rope_positions(x, {2, 5}, 10000.0f).as_f32();
    const std::vector<float> part = bk.apply_rope_partial(x, {2, 5}, 10000.0f, 8).as_f32();
    for (size_t i = 0; i < full.size(); ++i) ASSERT(std::fabs(full[i] - part[i]) < 1e-6f, "partial == full");
}

static void rope_position_zero_is_identity(HipLlmBackend& bk) {  // rope.rs:195-205
    const std::vector<float> data = {1.0f, 2.0f, 3.0f, 4.0f};
    const std::vector<float> o = bk.apply_rope_positions(Tensor::from_f32(data, {1, 1, 1, 4}), {0}, 10000.0f).as_f32();
    for (int i = 0; i < 4; ++i) ASSERT(std::fabs(o[i] - data[i]) < 1e-6f, "position 0 should be identity");
}

static void rope_rejects_bad_arguments(HipLlmBackend& bk) {  // rope.rs:19-35, :99-109
    const Tensor x3 = Tensor::from_f32(std::vector<float>(8, 1.0f), {1, 1, 8});
    ASSERT(expect_error([&] { bk.apply_rope_positions(x3, {0}, 1e4f); }).find("rank mismatch") != std::string::npos, "rank");
    const Tensor odd = Tensor::from_f32(std::vector<float>(5, 1.0f), {1, 1, 1, 5});
    ASSERT(expect_error([&] { bk.apply_rope_positions(odd, {0}, 1e4f); }).find("even head_dim") != std::string::npos, "odd");
    const Tensor x = Tensor::from_f32(std::vector<float>(16, 1.0f), {1, 1, 2, 8});
    ASSERT(expect_error([&] { bk.apply_rope_positions(x, {0}, 1e4f); }).find("positions length") != std::string::npos, "len");
    ASSERT(expect_error([&] { bk.apply_rope_partial(x, {0, 1}, 1e4f, 10); }).find("rotary_dim") != std::string::npos, "rd");
}

static void rope_table_and_device_angles_agree(HipLlmBackend& bk) {  // rope.rs:48-57
    // One call whose positions straddle the angle table's cap takes the device sin/cos path as a
    // whole; its tokens below the cap, rotated one call each, read the table (grown to them).
    // Both evaluate the reference's angle and its glibc sin/cos, so they agree bit for bit —
    // at positions near 2^18, where sinf/cosf take their large-argument reduction.
    const size_t H = 2, S = 40, D = 64, cap = HipLlmBackend::kRopeTableMaxRows;
    std::vector<float> x(H * S * D);
    for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(0.37f * (float)i) * 3.0f;
    std::vector<size_t> pos(S);
    for (size_t s = 0; s < S; ++s) pos[s] = cap - 20 + s;  // 20 below the cap, 20 at or past it
    const std::vector<float> all = bk.apply_rope_positions(Tensor::from_f32(x, {1, H, S, D}), pos, 5e5f).as_f32();
    for (size_t s = 0; s < 20; s += 3) {
        std::vector<float> one(H * D);
        for (size_t h = 0; h < H; ++h) std::memcpy(&one[h * D], &x[(h * S + s) * D], D * 4);
        const std::vector<float> o = bk.apply_rope_positions(Tensor::from_f32(one, {1, H, 1, D}), {pos[s]}, 5e5f).as_f32();
        for (size_t h = 0; h < H; ++h)
            ASSERT(std::memcmp(&o[h * D], &all[(h * S + s) * D], D * 4) == 0, "token rotated alike on both routes");
    }
    // A partial rotary on the same table machinery (another rotary_dim, another table): channels past
    // rotary_dim unchanged, and the rotated part equal to a full RoPE of a head of that width.
    std::vector<float> y(16);
    for (int i = 0; i < 16; ++i) y[i] = (float)(i + 1) * 0.25f;
    const std::vector<float> part = bk.apply_rope_partial(Tensor::from_f32(y, {1, 1, 1, 16}), {77}, 1e4f, 8).as_f32();
    const std::vector<float> head(y.begin(), y.begin() + 8);
    const std::vector<float> full = bk.apply_rope_positions(Tensor::from_f32(head, {1, 1, 1, 8}), {77}, 1e4f).as_f32();
    for (int i = 0; i < 8; ++i) ASSERT(std::memcmp(&part[i], &full[i], 4) == 0, "rotated part");
    for (int i = 8; i < 16; ++i) ASSERT(part[i] == y[i], "tail unchanged");
}

static void rope_interleaved_is_permuted_neox(HipLlmBackend& bk) {  // gguf_weights.rs:111-115
    const size_t D = 16;
    std::vector<float> x(2 * 3 * D);
    for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(0.37f * (float)i);
    std::vector<float> xp(x.size());
    for (size_t r = 0; r < x.size() / D; ++r)
        for (size_t c = 0; c < D; ++c) xp[r * D + c] = x[r * D + (c % 2) * (D / 2) + c / 2];
    const std::vector<float> n = bk.apply_rope_positions(Tensor::from_f32(x, {1, 2, 3, D}), {4, 9, 77}, 1e4f).as_f32();
    const std::vector<float> i = bk.apply_rope_interleaved(Tensor::from_f32(xp, {1, 2, 3, D}), {4, 9, 77}, 1e4f).as_f32();
    for (size_t r = 0; r < x.size() / D; ++r)
        for (size_t c = 0; c < D; ++c) ASSERT(i[r * D + c] == n[r * D + (c % 2) * (D / 2) + c / 2], "P neox(x)");
}

static void add_rms_norm_is_add_then_rms_norm(HipLlmBackend& bk) {  // llama.rs:508 → :515
    std::vector<float> a(3 * 64), b(3 * 64), w(64);
    for (size_t i = 0; i < a.size(); ++i) a[i] = std::cos(0.1f * (float)i), b[i] = std::sin(0.3f * (float)i);
    for (size_t i = 0; i < w.size(); ++i) w[i] = 1.0f + 0.01f * (float)i;
    const Tensor x = Tensor::from_f32(a, {3, 64}), r = Tensor::from_f32(b, {3, 64}), wt = Tensor::from_f32(w, {64});
    const auto fused = bk.add_rms_norm(x, r, wt, 1e-5f);
    const Tensor sum = bk.add(r, x);
    ASSERT(fused.second.as_f32() == sum.as_f32(), "residual == add");
    ASSERT(fused.first.as_f32() == bk.rms_norm(sum, wt, 1e-5f).as_f32(), "normed == rms_norm(add)");
}

static void embed_row_gather_matches_full_dequant(HipLlmBackend& bk) {  // common.rs:674-718
    const size_t vocab = 17, hidden = 256;
    uint64_t s = 0xABCD;
    std::vector<float> data(vocab * hidden);
    for (float& v : data) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        v = ((float)(s >> 40) / (float)(1u << 24)) * 2.0f - 1.0f;
    }
    const Tensor f32_t = Tensor::from_f32(data, {vocab, hidden});
    Bytes f16b;
    std::vector<float> f16_full;
    for (float v : data) {
        const uint16_t h = f16_from_f32(v);
        f16b.push_back((uint8_t)(h & 0xFF));
        f16b.push_back((uint8_t)(h >> 8));
        f16_full.push_back(f16_to_f32(h));
    }
    const Tensor f16_t = Tensor::from_f16_bytes(f16b, {vocab, hidden});
    const std::vector<uint8_t> q8 = quantize_q8_0(data);
    std::vector<float> q8_full;  // Tensor::to_f32_vec, Q8_0 arm (tensor.rs:378-389)
    for (size_t b = 0; b < q8.size() / 34; ++b) {
        const float d = f16_to_f32((uint16_t)(q8[b * 34] | (q8[b * 34 + 1] << 8)));
        for (int j = 0; j < 32; ++j) q8_full.push_back((float)(int8_t)q8[b * 34 + 2 + j] * d);
    }
    const Tensor q8_t = Tensor::from_quant_bytes(Bytes(q8.begin(), q8.end()), {vocab, hidden}, DType::Q8_0);
    const std::vector<uint32_t> ids = {0, 7, 16, 3};
    const std::pair<const Tensor*, const std::vector<float>*> tables[] = {{&f32_t, &data}, {&f16_t, &f16_full}, {&q8_t, &q8_full}};
    for (const auto& [table, full] : tables) {
        const Tensor got = bk.embed_tokens(*table, ids);
        ASSERT(got.shape() == std::vector<size_t>({1, ids.size(), hidden}), "shape [1, seq, hidden]");
        const std::vector<float> g = got.as_f32();
        for (size_t i = 0; i < ids.size(); ++i)
            ASSERT(std::memcmp(&g[i * hidden], &(*full)[ids[i] * hidden], hidden * 4) == 0,
                   std::string("row gather differs from full dequant (dtype ") + sapient_hip::dtype_name(table->dtype()) + ")");
    }
    // Out-of-range id still errors.
    const std::string e = expect_error([&] { bk.embed_tokens(f32_t, {(uint32_t)vocab}); });
    ASSERT(e.find("token id 17 out of vocab range") != std::string::npos, "OOR error");
}

// ── debug switches (SAPIENT_HIP_DISABLE / SAPIENT_HIP_VERIFY, after backend.rs:191-216) ──
// A stand-in for the caller's CPU backend: records each call and answers 7.0.
struct RecordingBackend : sapient_hip::LlmBackend {
    std::vector<std::string> calls;
    Tensor sevens(const Tensor& like) { return Tensor::from_f32(std::vector<float>(like.numel(), 7.0f), like.shape()); }
    Tensor hit(const char* op, const Tensor& like) {
        calls.push_back(op);
        return sevens(like);
    }
    const char* name() const override { return "recording"; }
    Tensor rms_norm(const Tensor& x, const Tensor&, float) override { return hit("rms_norm", x); }
    Tensor layer_norm(const Tensor& x, const Tensor&, const Tensor*, float) override { return hit("layer_norm", x); }
    Tensor add_bias_last_dim(const Tensor& y, const Tensor&) override { return hit("add_bias_last_dim", y); }
    Tensor silu(const Tensor& x) override { return hit("silu", x); }
    Tensor gelu(const Tensor& x) override { return hit("gelu", x); }
    Tensor gelu_erf(const Tensor& x) override { return hit("gelu_erf", x); }
    Tensor add(const Tensor& a, const Tensor&) override { return hit("add", a); }
    Tensor mul(const Tensor& a, const Tensor&) override { return hit("mul", a); }
    Tensor apply_rope_positions(const Tensor& x, const std::vector<size_t>&, float) override { return hit("rope", x); }
    Tensor apply_rope_partial(const Tensor& x, const std::vector<size_t>&, float, size_t) override {
        return hit("rope_partial", x);
    }
    Tensor apply_rope_interleaved(const Tensor& x, const std::vector<size_t>&, float) override {
        return hit("rope_interleaved", x);
    }
    Tensor embed_tokens(const Tensor& w, const std::vector<uint32_t>& ids) override {
        calls.push_back("embed_tokens");
        return Tensor::from_f32(std::vector<float>(ids.size() * w.shape()[1], 7.0f), {1, ids.size(), w.shape()[1]});
    }
};

// Sets an environment variable for one scope.
struct EnvVar {
    const char* name;
    EnvVar(const char* n, const char* v) : name(n) { setenv(n, v, 1); }
    ~EnvVar() { unsetenv(name); }
};

static bool all_sevens(const Tensor& t) {
    for (float v : t.as_f32())
        if (v != 7.0f) return false;
    return true;
}

static void disable_routes_listed_ops(HipLlmBackend&) {
    EnvVar env("SAPIENT_HIP_DISABLE", " RMS_norm, swiglu ,,rope");
    RecordingBackend cpu;
    HipLlmBackend bk(&cpu);
    ASSERT(bk.disabled("rms_norm") && bk.disabled("swiglu") && bk.disabled("rope") && !bk.disabled("silu"),
           "list parsed trimmed and lower-cased");
    const Tensor x = Tensor::from_f32({0.0f, 1.0f, -2.0f, 3.0f}, {1, 4});
    const Tensor w = Tensor::from_f32({1.0f, 1.0f, 1.0f, 1.0f}, {4});
    ASSERT(all_sevens(bk.rms_norm(x, w, 1e-5f)), "rms_norm answered by the given backend");
    ASSERT(cpu.calls == std::vector<std::string>({"rms_norm"}), "one rms_norm call");
    // swiglu goes to the given backend's default composition: mul(silu(gate), up).
    ASSERT(all_sevens(bk.swiglu(x, x)), "swiglu answered by the given backend");
    ASSERT(cpu.calls == std::vector<std::string>({"rms_norm", "silu", "mul"}), "swiglu via silu then mul");
    const Tensor q = Tensor::from_f32(std::vector<float>(8, 1.0f), {1, 1, 2, 4});
    ASSERT(all_sevens(bk.apply_rope_partial(q, {0, 1}, 1e4f, 2)), "every RoPE method is 'rope'");
    // Ops not listed stay on the device.
    const std::vector<float> s = bk.silu(x).as_f32();
    ASSERT(s[0] == 0.0f && s[1] > 0.73f && s[1] < 0.74f, "silu on the device");
    ASSERT(cpu.calls.size() == 4, "silu did not reach the given backend");
}

static void disable_without_backend_raises(HipLlmBackend&) {
    EnvVar env("SAPIENT_HIP_DISABLE", "all");
    HipLlmBackend bk;
    const Tensor a = Tensor::from_f32({1.0f, 2.0f}, {2});
    const std::string e = expect_error([&] { bk.add(a, a); });
    ASSERT(e.find("add: disabled by SAPIENT_HIP_DISABLE") != std::string::npos, "names op and switch: " + e);
}

static void verify_returns_the_device_result(HipLlmBackend&) {
    EnvVar env("SAPIENT_HIP_VERIFY", "1");
    RecordingBackend cpu;
    HipLlmBackend bk(&cpu);
    ASSERT(bk.verifying(), "switch read");
    const Tensor a = Tensor::from_f32({1.0f, 2.0f, 3.0f}, {3});
    const std::vector<float> sum = bk.add(a, a).as_f32();
    ASSERT(sum == std::vector<float>({2.0f, 4.0f, 6.0f}), "device result returned");
    ASSERT(cpu.calls == std::vector<std::string>({"add"}), "the given backend ran beside it");
    for (int i = 0; i < 70; ++i) (void)bk.mul(a, a);
    ASSERT(cpu.calls.size() == 64, "only the first 64 calls are cross-checked");
}

static void kv_cache_update_reference_test(HipLlmBackend& bk) {  // tests/inference_test.rs:10-61
    Tensor cache = Tensor::from_f32(std::vector<float>(16, 0.0f), {1, 2, 4, 2});
    const Tensor view1 = bk.update_kv_cache(cache, 0, Tensor::from_f32({1, 1, 2, 2}, {1, 2, 1, 2}));
    ASSERT((view1.shape() == std::vector<size_t>{1, 2, 1, 2}), "view after the first token");
    const Tensor view2 = bk.update_kv_cache(cache, 1, Tensor::from_f32({3, 3, 4, 4, 5, 5, 6, 6}, {1, 2, 2, 2}));
    ASSERT((view2.shape() == std::vector<size_t>{1, 2, 3, 2}), "view after two more");
    ASSERT((cache.as_f32() == std::vector<float>{1, 1, 3, 3, 4, 4, 0, 0, 2, 2, 5, 5, 6, 6, 0, 0}), "cache contents");
    ASSERT((view2.as_f32() == std::vector<float>{1, 1, 3, 3, 4, 4, 2, 2, 5, 5, 6, 6}), "view contents");
}

static void kv_cache_update_slides_when_full(HipLlmBackend& bk) {  // common.rs:381-412
    // Full cache (4 of 4 rows per head): one more token drops row 0; three more drop three.
    Tensor cache = Tensor::from_f32({1, 1, 2, 2, 3, 3, 4, 4, 11, 11, 12, 12, 13, 13, 14, 14}, {1, 2, 4, 2});
    const Tensor v = bk.update_kv_cache(cache, 4, Tensor::from_f32({5, 5, 15, 15}, {1, 2, 1, 2}));
    ASSERT((v.shape() == std::vector<size_t>{1, 2, 4, 2}), "view stays at max_seq");
    ASSERT((cache.as_f32() == std::vector<float>{2, 2, 3, 3, 4, 4, 5, 5, 12, 12, 13, 13, 14, 14, 15, 15}), "slid by one");
    (void)bk.update_kv_cache(cache, 3, Tensor::from_f32({6, 6, 7, 7, 8, 8, 16, 16, 17, 17, 18, 18}, {1, 2, 3, 2}));
    ASSERT((cache.as_f32() == std::vector<float>{4, 4, 6, 6, 7, 7, 8, 8, 14, 14, 16, 16, 17, 17, 18, 18}),
           "cur 3 + 3 new: two dropped, the kept row first");
    ASSERT(expect_error([&] { bk.update_kv_cache(cache, 4, Tensor::from_f32(std::vector<float>(20, 0.0f), {1, 2, 5, 2})); })
               .find("new tokens 5 exceeds max cache size 4") != std::string::npos, "too many new tokens");
    ASSERT(expect_error([&] { bk.update_kv_cache(cache, 0, Tensor::from_f32({1, 1, 1, 1}, {2, 1, 2})); })
               .find("expects 4-D tensors") != std::string::npos, "rank");
    ASSERT(expect_error([&] { bk.update_kv_cache(cache, 0, Tensor::from_f32({1, 1}, {1, 1, 1, 2})); })
               .find("shape mismatch") != std::string::npos, "heads");
}

static void kv_cache_update_refuses_half_caches(HipLlmBackend& bk) {  // common.rs:378 → tensor.rs:599-602
    // The float path writes through as_f32_slice_mut, which refuses every dtype but F32.
    Tensor cache = Tensor::from_f16_bytes(Bytes(32, 0), {1, 2, 4, 2});
    ASSERT(expect_error([&] { bk.update_kv_cache(cache, 0, Tensor::from_f32({1, 1, 2, 2}, {1, 2, 1, 2})); })
               .find("Tensor dtype is not F32") != std::string::npos, "f16 cache");
    Tensor cache_bf = Tensor::from_bf16_bytes(Bytes(32, 0), {1, 2, 4, 2});
    ASSERT(expect_error([&] { bk.update_kv_cache(cache_bf, 0, Tensor::from_f32({1, 1, 2, 2}, {1, 2, 1, 2})); })
               .find("Tensor dtype is not F32") != std::string::npos, "bf16 cache");
}

static void kv_cache_update_long_decode(HipLlmBackend& bk) {  // common.rs:381-412, step by step
    // Twelve one-token steps into a [1, 3, 5, 4] cache: the window slides from the sixth on; the
    // cache always holds the last min(t, 5) tokens of each head, oldest first.
    const size_t H = 3, S = 5, D = 4;
    Tensor cache = Tensor::from_f32(std::vector<float>(H * S * D, 0.0f), {1, H, S, D});
    size_t cur = 0;
    for (int t = 1; t <= 12; ++t) {
        std::vector<float> tok(H * D);
        for (size_t h = 0; h < H; ++h)
            for (size_t d = 0; d < D; ++d) tok[h * D + d] = (float)(100 * h + 10 * t) + (float)d;
        const Tensor v = bk.update_kv_cache(cache, cur, Tensor::from_f32(tok, {1, H, 1, D}));
        cur = v.shape()[2];
        ASSERT(cur == std::min<size_t>((size_t)t, S), "view length");
        const std::vector<float> c = cache.as_f32();
        for (size_t h = 0; h < H; ++h)
            for (size_t s = 0; s < cur; ++s) {
                const int tt = t - (int)cur + 1 + (int)s;
                for (size_t d = 0; d < D; ++d)
                    ASSERT(c[(h * S + s) * D + d] == (float)(100 * h + 10 * tt) + (float)d, "cache row");
            }
    }
}

static void kv_cache_update_q8_0(HipLlmBackend& bk) {  // update_kv_cache_q8, common.rs:449-528
    // [1, 1, 2, 32] Q8_0 cache holding one row; a full cache after a second, then a slide: rows are
    // quantized by quantize_f32_to_q8_0_block (common.rs:336-348, the quantizer of quant.rs:223-235),
    // moved as raw blocks, and the returned prefix is q · d in f32.
    std::vector<float> r0(32), r1(32), r2(32);
    for (int i = 0; i < 32; ++i) {
        r0[i] = (float)(i - 16) * 0.25f;
        r1[i] = std::sin((float)i);
        r2[i] = (float)(i % 5) - 2.0f;
    }
    std::vector<uint8_t> bytes = quantize_q8_0(r0);
    bytes.resize(68, 0);
    Tensor cache = Tensor::from_quant_bytes(Bytes(bytes.begin(), bytes.end()), {1, 1, 2, 32}, DType::Q8_0);
    const Tensor v1 = bk.update_kv_cache(cache, 1, Tensor::from_f32(r1, {1, 1, 1, 32}));
    std::vector<uint8_t> want = quantize_q8_0(r0), q1 = quantize_q8_0(r1);
    want.insert(want.end(), q1.begin(), q1.end());
    ASSERT(same_bytes(cache.bytes(), want), "second row quantized in place");
    const Tensor v2 = bk.update_kv_cache(cache, 2, Tensor::from_f32(r2, {1, 1, 1, 32}));
    std::vector<uint8_t> q2 = quantize_q8_0(r2);
    want.assign(q1.begin(), q1.end());
    want.insert(want.end(), q2.begin(), q2.end());
    ASSERT(same_bytes(cache.bytes(), want), "window slid by one block row");
    ASSERT((v2.shape() == std::vector<size_t>{1, 1, 2, 32}), "prefix shape");
    const std::vector<float> y = v2.as_f32();
    for (int s = 0; s < 2; ++s) {
        const uint8_t* blk = want.data() + 34 * s;
        const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < 32; ++i) ASSERT(y[32 * s + i] == (float)(int8_t)blk[2 + i] * d, "dequantized prefix");
    }
    (void)v1;
}

// Caches of 1 MiB or more are page-locked and updated where they lie (an append writes only the
// new rows; a slide moves the kept rows once into a fresh block that becomes the cache's storage):
// appends of 1 to 700 tokens into an F32 [1, 4, 1024, 128] and a Q8_0 [1, 8, 1024, 128] cache,
// sliding several times, each checked against the reference's update (common.rs:381-412,
// :449-528) restated on the host, cache bytes and returned prefix alike.
static void kv_cache_update_in_place_on_large_caches(HipLlmBackend& bk) {
    const size_t steps[] = {1, 1, 300, 1, 700, 50, 1, 1, 200, 1, 513, 1, 1024, 3};
    for (const bool q8 : {false, true}) {
        const size_t H = q8 ? 8 : 4, S = 1024, D = 128;
        const size_t row = q8 ? D / 32 * 34 : D * 4;  // bytes per cache row
        std::vector<uint8_t> want(H * S * row, 0);
        Tensor cache = q8 ? Tensor::from_quant_bytes(Bytes(want.size(), 0), {1, H, S, D}, DType::Q8_0)
                          : Tensor::from_f32(std::vector<float>(H * S * D, 0.0f), {1, H, S, D});
        size_t cur = 0, t = 0;
        for (size_t ns : steps) {
            std::vector<float> nk(H * ns * D);
            for (size_t i = 0; i < nk.size(); ++i) nk[i] = (float)(int)((i * 7 + t * 131) % 2001) * 0.01f - 10.0f;
            t += ns;
            const Tensor view = bk.update_kv_cache(cache, cur, Tensor::from_f32(nk, {1, H, ns, D}));
            const size_t shift = cur + ns > S ? cur + ns - S : 0, keep = cur - shift;
            for (size_t hh = 0; hh < H; ++hh) {
                uint8_t* base = want.data() + hh * S * row;
                std::memmove(base, base + shift * row, keep * row);
                for (size_t s = 0; s < ns; ++s) {
                    const float* src = nk.data() + (hh * ns + s) * D;
                    if (q8) {
                        const std::vector<uint8_t> q = quantize_q8_0(std::vector<float>(src, src + D));
                        std::memcpy(base + (keep + s) * row, q.data(), row);
                    } else {
                        std::memcpy(base + (keep + s) * row, src, row);
                    }
                }
            }
            cur = std::min(S, cur + ns);
            ASSERT(view.shape()[2] == cur, "prefix length");
            ASSERT(same_bytes(cache.bytes(), want), q8 ? "q8_0 cache bytes" : "f32 cache bytes");
            const std::vector<float> got = view.as_f32();
            for (size_t hh = 0; hh < H; ++hh)
                for (size_t s = 0; s < cur; ++s) {
                    const uint8_t* r = want.data() + (hh * S + s) * row;
                    for (size_t d = 0; d < D; ++d) {
                        float v;
                        if (q8) {
                            const uint8_t* blk = r + d / 32 * 34;
                            v = (float)(int8_t)blk[2 + d % 32] * f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                        } else {
                            std::memcpy(&v, r + d * 4, 4);
                        }
                        if (std::memcmp(&v, &got[(hh * cur + s) * D + d], 4) != 0) throw Failure{"prefix value"};
                    }
                }
        }
    }
}

static void quant_bytes_are_validated(HipLlmBackend&) {  // tensor.rs:143-169
    ASSERT(expect_error([] { Tensor::from_quant_bytes(Bytes(33), {32}, DType::Q8_0); })
               .find("shape mismatch") != std::string::npos, "byte count");
}

// Copies share one byte buffer (the reference's Arc'd buffer): no bytes are copied until one copy
// writes (Arc::make_mut), and then only that copy changes; a reshape shares them too. An op's
// result owns fresh bytes, and a kv-cache update writes only the tensor it is given.
static void tensor_copies_share_bytes_until_written(HipLlmBackend& bk) {
    const Tensor a = Tensor::from_f32({1, 2, 3, 4}, {2, 2});
    Tensor b = a;
    const Tensor c = a.reshaped({4});
    ASSERT(b.bytes().data() == a.bytes().data() && c.bytes().data() == a.bytes().data(), "copies share bytes");
    float nine = 9.0f;
    std::memcpy(b.bytes_mut().data(), &nine, 4);
    ASSERT(b.bytes().data() != a.bytes().data(), "a write gives the copy its own bytes");
    ASSERT(a.as_f32()[0] == 1.0f && c.as_f32()[0] == 1.0f && b.as_f32()[0] == 9.0f, "only the written copy changed");
    ASSERT(b.as_f32()[3] == 4.0f, "the rest copied");
    const Tensor s = bk.silu(a);
    ASSERT(s.bytes().data() != a.bytes().data() && a.as_f32()[1] == 2.0f, "an op's result owns fresh bytes");
    // update_kv_cache writes the cache it is given in place, not a copy sharing its bytes
    Tensor cache = Tensor::from_f32(std::vector<float>(1 * 1 * 4 * 2, 0.0f), {1, 1, 4, 2});
    const Tensor kept = cache;
    (void)bk.update_kv_cache(cache, 0, Tensor::from_f32({5, 6}, {1, 1, 1, 2}));
    ASSERT(cache.as_f32()[0] == 5.0f && cache.as_f32()[1] == 6.0f, "cache row 0 written");
    ASSERT(kept.as_f32()[0] == 0.0f && kept.as_f32()[1] == 0.0f, "the earlier copy keeps its bytes");
}

// Tensor bytes of 1 MiB or more are page-locked host memory (so transfers run as direct DMA), and a
// dropped tensor's block goes to the next one of a fitting size, pages already mapped; a live
// tensor's bytes are never handed out again, and a result outlives the backend that made it.
static bool page_locked(const void* p) {
    hipPointerAttribute_t a{};
    const bool yes = hipPointerGetAttributes(&a, p) == hipSuccess && a.type == hipMemoryTypeHost;
    (void)hipGetLastError();  // plain heap memory is an error to the query
    return yes;
}

static void large_tensor_bytes_are_page_locked_and_recycled(HipLlmBackend& bk) {
    const size_t n = size_t(1) << 19;  // 2 MiB of f32
    std::vector<float> xs(n);
    for (size_t i = 0; i < n; ++i) xs[i] = (float)(int)(i % 97) * 0.125f - 6.0f;
    const Tensor x = Tensor::from_f32(xs, {n});
    ASSERT(page_locked(x.bytes().data()), "a large input tensor's bytes are page-locked");
    const uint8_t* first = nullptr;
    std::vector<float> want;
    {
        const Tensor a = bk.silu(x);
        ASSERT(page_locked(a.bytes().data()), "a large result's bytes are page-locked");
        first = a.bytes().data();
        want = a.as_f32();
    }
    const Tensor b = bk.silu(x);
    ASSERT(b.bytes().data() == first, "a dropped result's block is reused");
    ASSERT(b.as_f32() == want, "the reused block holds the new result");
    const Tensor c = bk.gelu(x);
    ASSERT(c.bytes().data() != b.bytes().data(), "a live result's block is not handed out");
    const Tensor small = bk.silu(Tensor::from_f32({1.0f, -2.0f}, {2}));
    ASSERT(!page_locked(small.bytes().data()), "small tensors are plain heap memory");
    Bytes grown{1, 2, 3, 4, 5, 6, 7, 8};
    grown.resize(size_t(3) << 20);  // reallocated into a large block
    ASSERT(page_locked(grown.data()), "a grown byte buffer is page-locked");
    ASSERT(grown[0] == 1 && grown[7] == 8, "growing keeps the contents");
    Tensor kept;
    {
        HipLlmBackend other;
        kept = other.silu(x);
    }
    ASSERT(kept.as_f32() == want, "a result outlives its backend");
}

// Large tensors (page-locked bytes) are read and written by the kernels in place, over the host
// link; small ones go through device buffers. Every row of a large call must be what a small call
// on those rows gives: bit for bit for the element-wise ops, the bias, RoPE, the gather and the
// residual sum, and within 1e-5 relative for the normalized rows (the row reduction's order can
// follow the launch shape).
static Tensor rows_of(const Tensor& t, size_t r0, size_t n) {
    std::vector<size_t> shape = t.shape();
    const size_t row = t.numel() / shape[0];
    shape[0] = n;
    const size_t rb = byte_count(t.dtype(), row);
    Bytes b(t.bytes().begin() + r0 * rb, t.bytes().begin() + (r0 + n) * rb);
    return t.dtype() == DType::F32 ? Tensor::from_f32_bytes(std::move(b), shape)
                                   : Tensor::from_quant_bytes(std::move(b), shape, t.dtype());
}

static bool rows_match(const Tensor& big, size_t r0, const Tensor& part, float rel) {
    const std::vector<float> a = big.as_f32(), b = part.as_f32();
    const size_t row = big.numel() / big.shape()[0];
    for (size_t i = 0; i < b.size(); ++i) {
        const float x = a[r0 * row + i], y = b[i];
        if (rel == 0.0f ? std::memcmp(&x, &y, 4) != 0 : std::fabs(x - y) > rel * std::max(1.0f, std::fabs(y))) return false;
    }
    return true;
}

static void large_calls_equal_small_calls(HipLlmBackend& bk) {
    const size_t R = 4096, D = 2048;  // 32 MiB per f32 operand: several chunks
    std::vector<float> xv(R * D), rv(R * D), wv(D), bv(D);
    uint64_t st = 0x9E3779B97F4A7C15ull;
    auto rnd = [&] {
        st = st * 6364136223846793005ull + 1442695040888963407ull;
        return ((float)(st >> 40) / (float)(1u << 24)) * 4.0f - 2.0f;
    };
    for (auto& v : xv) v = rnd();
    for (auto& v : rv) v = rnd();
    for (auto& v : wv) v = 1.0f + 0.1f * rnd();
    for (auto& v : bv) v = rnd();
    const Tensor x = Tensor::from_f32(xv, {R, D}), r = Tensor::from_f32(rv, {R, D});
    const Tensor w = Tensor::from_f32(wv, {D}), b = Tensor::from_f32(bv, {D});
    const Tensor two = Tensor::from_f32({2.5f}, {1});
    const size_t S = 8, HD = 128, NH = R * D / (S * HD);  // RoPE over 8192 heads of 8 x 128
    std::vector<size_t> positions(S);
    for (size_t i = 0; i < S; ++i) positions[i] = 1000 + 37 * i;
    const auto ar = bk.add_rms_norm(x, r, w, 1e-5f);
    const Tensor rn = bk.rms_norm(x, w, 1e-5f), ln = bk.layer_norm(x, w, &b, 1e-5f);
    const Tensor si = bk.silu(x), ge = bk.gelu(x), ml = bk.mul(x, two), ad = bk.add(x, r), sw = bk.swiglu(x, r);
    const Tensor bi = bk.add_bias_last_dim(x, b);
    const Tensor ro = bk.apply_rope_positions(x.reshaped({1, NH, S, HD}), positions, 10000.0f).reshaped({NH, S * HD});
    const size_t slices[][2] = {{0, 10}, {1000, 100}, {2040, 16}, {R - 6, 6}};
    for (const auto& sl : slices) {
        const size_t r0 = sl[0], n = sl[1];
        const Tensor xs = rows_of(x, r0, n), rs = rows_of(r, r0, n);
        const auto p = bk.add_rms_norm(xs, rs, w, 1e-5f);
        ASSERT(rows_match(ar.second, r0, p.second, 0.0f), "add_rms_norm sum");
        ASSERT(rows_match(ar.first, r0, p.first, 1e-5f), "add_rms_norm normed");
        ASSERT(rows_match(rn, r0, bk.rms_norm(xs, w, 1e-5f), 1e-5f), "rms_norm");
        ASSERT(rows_match(ln, r0, bk.layer_norm(xs, w, &b, 1e-5f), 1e-5f), "layer_norm");
        ASSERT(rows_match(si, r0, bk.silu(xs), 0.0f), "silu");
        ASSERT(rows_match(ge, r0, bk.gelu(xs), 0.0f), "gelu");
        ASSERT(rows_match(ml, r0, bk.mul(xs, two), 0.0f), "mul by a length-1 side");
        ASSERT(rows_match(ad, r0, bk.add(xs, rs), 0.0f), "add");
        ASSERT(rows_match(sw, r0, bk.swiglu(xs, rs), 0.0f), "swiglu");
        ASSERT(rows_match(bi, r0, bk.add_bias_last_dim(xs, b), 0.0f), "add_bias_last_dim");
    }
    for (const auto& sl : {std::pair<size_t, size_t>{0, 10}, {4090, 16}, {NH - 6, 6}}) {
        const Tensor heads = rows_of(x.reshaped({NH, S * HD}), sl.first, sl.second).reshaped({1, sl.second, S, HD});
        const Tensor rot = bk.apply_rope_positions(heads, positions, 10000.0f).reshaped({sl.second, S * HD});
        ASSERT(rows_match(ro, sl.first, rot, 0.0f), "rope");
    }
    // the gather: 70000 ids of a 4096 x 64 Q8_0 table (17.9 MB of output; the table itself, 278 KB,
    // goes through a device buffer) and of a 65536 x 64 one read in place (4.5 MB)
    const size_t V = 4096, H = 64, N = 70000;
    std::vector<float> tv(V * H);
    for (auto& v : tv) v = rnd();
    const std::vector<uint8_t> q8 = quantize_q8_0(tv);
    const Tensor table = Tensor::from_quant_bytes(Bytes(q8.begin(), q8.end()), {V, H}, DType::Q8_0);
    std::vector<uint32_t> ids(N);
    for (size_t i = 0; i < N; ++i) ids[i] = (uint32_t)((i * 2654435761u) % V);
    const Tensor all = bk.embed_tokens(table, ids).reshaped({N, H});
    for (size_t i0 : {size_t(0), size_t(34000), N - 5}) {
        const std::vector<uint32_t> part(ids.begin() + i0, ids.begin() + std::min(N, i0 + 200));
        ASSERT(rows_match(all, i0, bk.embed_tokens(table, part).reshaped({part.size(), H}), 0.0f), "embed_tokens");
    }
    const size_t V2 = 65536;
    std::vector<float> tv2(V2 * H);
    for (auto& v : tv2) v = rnd();
    const std::vector<uint8_t> q82 = quantize_q8_0(tv2);
    const Tensor big_table = Tensor::from_quant_bytes(Bytes(q82.begin(), q82.end()), {V2, H}, DType::Q8_0);
    const Tensor small_table = rows_of(big_table, V2 - 4096, 4096);  // 278 KB: through a device buffer
    std::vector<uint32_t> hi(300), lo(300);
    for (size_t i = 0; i < hi.size(); ++i) {
        lo[i] = (uint32_t)((i * 40503u) % 4096);
        hi[i] = (uint32_t)(V2 - 4096) + lo[i];
    }
    ASSERT(rows_match(bk.embed_tokens(big_table, hi).reshaped({hi.size(), H}), 0,
                      bk.embed_tokens(small_table, lo).reshaped({lo.size(), H}), 0.0f),
           "embed_tokens from a table read in place");
}

// Threads share the process-wide cache of page-locked blocks and, when they share a backend, its
// staging (calls serialise on the backend's lock): four threads, two on a shared backend and two on
// backends of their own, each run large (in place) and small (staged) calls on their own data many
// times; every result must equal the single-threaded one, bit for bit.
static void threads_share_blocks_and_staging(HipLlmBackend& shared) {
    const size_t big = size_t(1) << 19, small = 4096;  // 2 MiB and 16 KiB of f32
    auto make = [](size_t n, int seed) {
        std::vector<float> v(n);
        for (size_t i = 0; i < n; ++i) v[i] = (float)(int)((i * 2654435761u + (size_t)seed * 97u) % 4001) * 0.001f - 2.0f;
        return v;
    };
    struct Case {
        Tensor xb, rb, xs, rs, w;
    };
    std::vector<Case> cases;
    for (int t = 0; t < 4; ++t)
        cases.push_back({Tensor::from_f32(make(big, t), {big / 4096, 4096}), Tensor::from_f32(make(big, t + 10), {big / 4096, 4096}),
                         Tensor::from_f32(make(small, t + 20), {1, small}), Tensor::from_f32(make(small, t + 30), {1, small}),
                         Tensor::from_f32(make(4096, 40), {4096})});
    auto run = [](HipLlmBackend& bk, const Case& c) {
        std::vector<std::vector<float>> out;
        const auto p = bk.add_rms_norm(c.xb, c.rb, c.w, 1e-5f);
        out.push_back(p.first.as_f32());
        out.push_back(p.second.as_f32());
        out.push_back(bk.silu(c.xb).as_f32());
        out.push_back(bk.add(c.xs, c.rs).as_f32());
        out.push_back(bk.swiglu(c.xs, c.rs).as_f32());
        out.push_back(bk.rms_norm(c.xs.reshaped({1, small}), Tensor::from_f32(std::vector<float>(small, 1.0f), {small}), 1e-6f).as_f32());
        return out;
    };
    std::vector<std::vector<std::vector<float>>> want;
    for (const Case& c : cases) want.push_back(run(shared, c));
    std::vector<std::string> errors(4);
    std::vector<std::thread> threads;
    for (int t = 0; t < 4; ++t)
        threads.emplace_back([&, t] {
            try {
                std::unique_ptr<HipLlmBackend> own;
                if (t >= 2) own = std::make_unique<HipLlmBackend>();
                HipLlmBackend& bk = own ? *own : shared;
                for (int round = 0; round < 10; ++round)
                    if (run(bk, cases[t]) != want[t]) {
                        errors[t] = "thread " + std::to_string(t) + " round " + std::to_string(round) + " differs";
                        return;
                    }
            } catch (const std::exception& e) {
                errors[t] = e.what();
            }
        });
    for (auto& th : threads) th.join();
    for (const std::string& e : errors) ASSERT(e.empty(), e);
}

int main() {
    if (!HipLlmBackend::is_available()) {
        std::printf("no gfx950 device\n");
        return 1;
    }
    HipLlmBackend bk;
    const std::pair<const char*, void (*)(HipLlmBackend&)> tests[] = {
        {"rmsnorm_identity_weight", rmsnorm_identity_weight},
        {"rmsnorm_half_input_outputs_f32", rmsnorm_half_input_outputs_f32},
        {"layernorm_zero_mean_unit_var", layernorm_zero_mean_unit_var},
        {"test_gelu_erf", test_gelu_erf},
        {"add_bias_last_dim_broadcasts", add_bias_last_dim_broadcasts},
        {"graph_rms_norm_optional_weight", graph_rms_norm_optional_weight},
        {"graph_layer_norm_axis", graph_layer_norm_axis},
        {"graph_embedding_ids_and_shape", graph_embedding_ids_and_shape},
        {"graph_rope_positions_from_seq", graph_rope_positions_from_seq},
        {"test_add", test_add},
        {"test_scalar_broadcast", test_scalar_broadcast},
        {"test_gelu", test_gelu},
        {"test_silu_and_swiglu", test_silu_and_swiglu},
        {"unary_rejects_non_f32", unary_rejects_non_f32},
        {"rope_output_shape", rope_output_shape},
        {"rope_partial_leaves_tail_unchanged", rope_partial_leaves_tail_unchanged},
        {"rope_partial_full_matches_apply_rope", rope_partial_full_matches_apply_rope},
        {"rope_position_zero_is_identity", rope_position_zero_is_identity},
        {"rope_rejects_bad_arguments", rope_rejects_bad_arguments},
        {"rope_interleaved_is_permuted_neox", rope_interleaved_is_permuted_neox},
        {"rope_table_and_device_angles_agree", rope_table_and_device_angles_agree},
        {"add_rms_norm_is_add_then_rms_norm", add_rms_norm_is_add_then_rms_norm},
        {"embed_row_gather_matches_full_dequant", embed_row_gather_matches_full_dequant},
        {"quant_bytes_are_validated", quant_bytes_are_validated},
        {"tensor_copies_share_bytes_until_written", tensor_copies_share_bytes_until_written},
        {"large_tensor_bytes_are_page_locked_and_recycled", large_tensor_bytes_are_page_locked_and_recycled},
        {"large_calls_equal_small_calls", large_calls_equal_small_calls},
        {"threads_share_blocks_and_staging", threads_share_blocks_and_staging},
        {"kv_cache_update_reference_test", kv_cache_update_reference_test},
        {"kv_cache_update_slides_when_full", kv_cache_update_slides_when_full},
        {"kv_cache_update_q8_0", kv_cache_update_q8_0},
        {"kv_cache_update_refuses_half_caches", kv_cache_update_refuses_half_caches},
        {"kv_cache_update_long_decode", kv_cache_update_long_decode},
        {"kv_cache_update_in_place_on_large_caches", kv_cache_update_in_place_on_large_caches},
        {"disable_routes_listed_ops", disable_routes_listed_ops},
        {"disable_without_backend_raises", disable_without_backend_raises},
        {"verify_returns_the_device_result", verify_returns_the_device_result},
    };
    int failed = 0;
    for (const auto& [name, fn] : tests) {
        std::printf("test %s ... ", name);
        std::fflush(stdout);
        try {
            fn(bk);
            std::printf("ok\n");
        } catch (const Failure& f) {
            std::printf("FAILED: %s\n", f.why.c_str());
            ++failed;
        } catch (const std::exception& e) {
            std::printf("FAILED (exception): %s\n", e.what());
            ++failed;
        }
        std::fflush(stdout);
    }
    std::printf("%d failed\n", failed);
    return failed ? 1 : 0;
}
