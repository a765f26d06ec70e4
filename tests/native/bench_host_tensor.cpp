// bench_host_tensor.cpp — the host-tensor rate of the C++ LlmBackend mirror
// (include/sapient_hip_backend.hpp), which bench.py runs as a child process and
// reports beside its device-resident figures: the fused residual add + RMSNorm
// on 16384 x 4096 f32 HOST tensors (the trait's calling convention,
// crates/sapient-models/src/forward/backend.rs:57-115: inputs and results in
// host memory, so every call crosses the host link both ways), the same call
// on one 4096-wide row (a decode step), and the embedding gather of one token
// id from a 128256 x 4096 Q8_0 host table.
// Prints one JSON line: {"host_tensor": {...}} (null with a reason when no
// gfx950 device answers).
#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <vector>

#include "sapient_hip_backend.hpp"

using sapient_hip::Bytes;
using sapient_hip::DType;
using sapient_hip::HipLlmBackend;
using sapient_hip::Tensor;

static std::vector<float> xv1(size_t n) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = (float)(int)((i * 2654435761u) % 2001) * 0.001f - 1.0f;
    return v;
}

template <typename F>
static double ms_of(F&& f) {
    const auto t0 = std::chrono::steady_clock::now();
    f();
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

static double median(std::vector<double> v) {
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

int main() {
    if (!HipLlmBackend::is_available()) {
        std::printf("{\"host_tensor\": null, \"reason\": \"no gfx950 device\"}\n");
        return 0;
    }
    const size_t R = 16384, D = 4096;
    uint64_t s = 0x243F6A8885A308D3ull;
    auto next = [&] {  // uniform in [-1, 1)
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        return (float)(int32_t)(s >> 32) * 0x1p-31f;
    };
    std::vector<float> xv(R * D), rv(R * D), wv(D);
    for (auto& v : xv) v = next();
    for (auto& v : rv) v = next();
    for (auto& v : wv) v = 1.0f + 0.1f * next();
    const Tensor x = Tensor::from_f32(xv, {R, D}), r = Tensor::from_f32(rv, {R, D}), w = Tensor::from_f32(wv, {D});
    xv = {};
    rv = {};
    HipLlmBackend bk;
    const double alg = 4.0 * R * D * 4 + D * 4;
    const double first = ms_of([&] { (void)bk.add_rms_norm(x, r, w, 1e-5f); });
    std::vector<double> t;
    for (int i = 0; i < 7; ++i) t.push_back(ms_of([&] { (void)bk.add_rms_norm(x, r, w, 1e-5f); }));
    const double ms = median(t);

    const size_t V = 128256, H = 4096;
    Bytes tb(V * H / 32 * 34);
    for (size_t b = 0; b < V * H / 32; ++b) {
        tb[34 * b] = 0x00;
        tb[34 * b + 1] = 0x1c;  // d = 2^-8 (f16)
        for (int j = 0; j < 32; ++j) tb[34 * b + 2 + j] = (uint8_t)((b * 7 + (size_t)j * 13) & 0xFF);
    }
    // a decode step's fused add + RMSNorm: one 4096-wide row (operands through page-locked staging)
    const Tensor x1 = Tensor::from_f32(std::vector<float>(xv1(D)), {1, D});
    const Tensor r1 = Tensor::from_f32(std::vector<float>(xv1(D)), {1, D});
    for (int i = 0; i < 5; ++i) (void)bk.add_rms_norm(x1, r1, w, 1e-5f);
    std::vector<double> td;
    for (int i = 0; i < 51; ++i) td.push_back(ms_of([&] { (void)bk.add_rms_norm(x1, r1, w, 1e-5f); }));

    const Tensor table = Tensor::from_quant_bytes(std::move(tb), {V, H}, DType::Q8_0);
    const std::vector<uint32_t> one = {12345};
    (void)bk.embed_tokens(table, one);
    std::vector<double> te;
    for (int i = 0; i < 7; ++i) te.push_back(ms_of([&] { (void)bk.embed_tokens(table, one); }));

    std::printf("{\"host_tensor\": {\"op\": \"add_rms_norm\", \"shape\": \"16384x4096 f32\", \"ms\": %.3f, "
                "\"GB/s\": %.1f, \"first_call_ms\": %.2f, \"embed_one_id_ms\": %.4f, \"decode_row_us\": %.1f, "
                "\"how\": \"C++ LlmBackend mirror on host tensors: page-locked bytes read and written in place "
                "by the kernels over the host link (medians: 7 calls after one; the decode row 51 after 5)\"}}\n",
                ms, alg / ms / 1e6, first, median(te), median(td) * 1e3);
    return 0;
}
