// Host-side tests of the C++ mirror's Tensor and its byte storage
// (include/sapient_hip_backend.hpp), runnable without a GPU: the data model of
// sapient_core::Tensor (crates/sapient-core/src/tensor.rs:22-29, :51-71,
// :143-169) — shapes and byte counts validated at construction, copies sharing
// one refcounted buffer until one of them writes (buffer.rs:54) — and the
// byte counts of dtype.rs:136-145. Prints "test <name> ... ok|FAILED: <why>";
// exits 1 if any failed.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "sapient_hip_backend.hpp"

using sapient_hip::byte_count;
using sapient_hip::Bytes;
using sapient_hip::DType;
using sapient_hip::Error;
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

static void shapes_and_byte_counts_are_validated() {
    ASSERT(expect_error([] { Tensor::from_f32({1, 2, 3}, {2, 2}); }).find("shape mismatch") != std::string::npos,
           "from_f32");
    ASSERT(expect_error([] { Tensor::from_f32_bytes(Bytes(12), {2, 2}); }).find("shape mismatch") != std::string::npos,
           "from_f32_bytes");
    ASSERT(expect_error([] { Tensor::from_f16_bytes(Bytes(6), {2, 2}); }).find("shape mismatch") != std::string::npos,
           "from_f16_bytes");
    ASSERT(expect_error([] { Tensor::from_quant_bytes(Bytes(33), {32}, DType::Q8_0); }).find("shape mismatch") !=
               std::string::npos,
           "q8_0 bytes");
    ASSERT(expect_error([] { Tensor::from_quant_bytes(Bytes(4), {2}, DType::F16); }).find("type mismatch") !=
               std::string::npos,
           "not a quantized dtype");
    const Tensor t = Tensor::from_f32({1, 2, 3, 4, 5, 6}, {2, 3});
    ASSERT(expect_error([&] { (void)t.reshaped({4, 2}); }).find("cannot reshape") != std::string::npos, "reshape");
    ASSERT(expect_error([] { (void)Tensor::from_f16_bytes(Bytes(4, 0), {2}).as_f32(); }).find("type mismatch") !=
               std::string::npos,
           "as_f32 of f16");
}

static void byte_counts_follow_the_block_formats() {  // dtype.rs:136-145
    ASSERT(byte_count(DType::F32, 10) == 40 && byte_count(DType::F16, 10) == 20 && byte_count(DType::BF16, 10) == 20,
           "floats");
    ASSERT(byte_count(DType::Q4_0, 64) == 36 && byte_count(DType::Q8_0, 64) == 68, "32-element blocks");
    ASSERT(byte_count(DType::Q4_K, 512) == 288 && byte_count(DType::Q5_K, 256) == 176 &&
               byte_count(DType::Q6_K, 256) == 210,
           "256-element blocks");
}

static void copies_share_bytes_until_one_writes() {
    const Tensor a = Tensor::from_f32({1, 2, 3, 4}, {2, 2});
    Tensor b = a;
    const Tensor c = a.reshaped({4});
    ASSERT(b.bytes().data() == a.bytes().data() && c.bytes().data() == a.bytes().data(), "shared");
    const float nine = 9.0f;
    std::memcpy(b.bytes_mut().data() + 4, &nine, 4);
    ASSERT(b.bytes().data() != a.bytes().data(), "a write detaches the writer");
    ASSERT(a.as_f32()[1] == 2.0f && c.as_f32()[1] == 2.0f && b.as_f32()[1] == 9.0f, "only the writer changed");
    Tensor d = Tensor::from_f32({5, 6}, {2});
    const uint8_t* before = d.bytes().data();
    (void)d.bytes_mut();
    ASSERT(d.bytes().data() == before, "an unshared tensor writes in place");
}

static void byte_storage_grows_and_keeps_its_contents() {
    // Large blocks (page-locked where a device answers, plain heap here) and small ones behave as a vector.
    Bytes v{1, 2, 3};
    v.resize(size_t(3) << 20);
    ASSERT(v[0] == 1 && v[2] == 3, "contents kept across growth into a large block");
    v.resize(5);
    ASSERT(v.size() == 5 && v[1] == 2, "shrinking keeps the front");
    Bytes filled(size_t(2) << 20, 7);
    ASSERT(filled[0] == 7 && filled[filled.size() - 1] == 7, "a fill value fills");
    std::vector<Bytes> many;
    for (int i = 0; i < 8; ++i) many.emplace_back(size_t(1) << 20, (uint8_t)i);
    for (int i = 0; i < 8; ++i) ASSERT(many[i][12345] == (uint8_t)i, "distinct large blocks");
    many.clear();  // back to the process-wide cache
    const Tensor big = Tensor::from_f32(std::vector<float>(size_t(1) << 19, 1.5f), {size_t(1) << 19});
    ASSERT(big.as_f32()[(size_t(1) << 19) - 1] == 1.5f, "a large tensor round-trips");
}

int main() {
    const std::pair<const char*, void (*)()> tests[] = {
        {"shapes_and_byte_counts_are_validated", shapes_and_byte_counts_are_validated},
        {"byte_counts_follow_the_block_formats", byte_counts_follow_the_block_formats},
        {"copies_share_bytes_until_one_writes", copies_share_bytes_until_one_writes},
        {"byte_storage_grows_and_keeps_its_contents", byte_storage_grows_and_keeps_its_contents},
    };
    int failed = 0;
    for (const auto& [name, fn] : tests) {
        try {
            fn();
            std::printf("test %s ... ok\n", name);
        } catch (const Failure& f) {
            std::printf("test %s ... FAILED: %s\n", name, f.why.c_str());
            ++failed;
        } catch (const std::exception& e) {
            std::printf("test %s ... FAILED: exception %s\n", name, e.what());
            ++failed;
        }
    }
    std::printf("%d failed\n", failed);
    return failed ? 1 : 0;
}
