// sapient_hip_backend.hpp — C++ host-side mirror of sapient's LlmBackend op
// surface on the MI355X kernels of sapient_hip.h.
//
// The reference trait (crates/sapient-models/src/forward/backend.rs:57-115)
// takes host tensors and returns new host tensors; this class does the same —
// the HIP kernels, through the C ABI on its own stream, read the inputs and
// write the results in host memory (page-locked bytes in place, small ones
// through page-locked staging) — with the reference's argument meaning,
// validation and error messages. It is
// what a Rust `HipLlmBackend` wrapper does over FFI, written in C++ because the
// reference is compiled code. There is no CPU fallback: a failed HIP call
// raises sapient_hip::Error (the debug switches below route an op elsewhere
// only when the caller asks for it).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "sapient_hip.h"

namespace sapient_hip {

// Tensor dtypes of the op set (values are GGUF type ids, as in sapient_hip.h).
enum class DType : int {
    F32 = SPH_F32, F16 = SPH_F16, BF16 = SPH_BF16, Q4_0 = SPH_Q4_0, Q8_0 = SPH_Q8_0, Q4_K = SPH_Q4_K, Q5_K = SPH_Q5_K,
    Q6_K = SPH_Q6_K
};

const char* dtype_name(DType dt);
bool is_quantized(DType dt);
// Bytes of `numel` elements (crates/sapient-core/src/dtype.rs:136-145).
size_t byte_count(DType dt, size_t numel);

class Error : public std::runtime_error {
 public:
    using std::runtime_error::runtime_error;
};

// Host memory for tensor bytes. Blocks of 1 MiB or more are page-locked
// (hipHostMalloc) when a HIP device is present, so the kernels read and write
// them in place through their device mapping (and any copy of them runs as
// direct DMA, ~4.7 ms per 256 MiB each way, rather than through the runtime's
// staging of pageable memory, 9-21 ms), and are kept for reuse when freed (up
// to 4 GiB in all, process-wide): a freed block goes to the next request
// needing between half and all of it, most recently freed first, with its
// pages already mapped. Smaller blocks are plain heap memory.
void* host_bytes_alloc(size_t n);
void host_bytes_free(void* p, size_t n) noexcept;

// The allocator of Bytes. Growing a Bytes without a fill value leaves the
// new bytes uninitialised (as Vec::with_capacity + set_len would): a tensor's
// bytes are always written in full before they are read.
template <typename T>
struct HostAlloc {
    using value_type = T;
    HostAlloc() noexcept = default;
    template <typename U>
    HostAlloc(const HostAlloc<U>&) noexcept {}
    T* allocate(size_t n) { return static_cast<T*>(host_bytes_alloc(n * sizeof(T))); }
    void deallocate(T* p, size_t n) noexcept { host_bytes_free(p, n * sizeof(T)); }
    template <typename U>
    void construct(U* p) noexcept {
        ::new (static_cast<void*>(p)) U;
    }
    template <typename U, typename... A>
    void construct(U* p, A&&... a) {
        ::new (static_cast<void*>(p)) U(std::forward<A>(a)...);
    }
    friend bool operator==(const HostAlloc&, const HostAlloc&) { return true; }
    friend bool operator!=(const HostAlloc&, const HostAlloc&) { return false; }
};

// A tensor's little-endian bytes.
using Bytes = std::vector<uint8_t, HostAlloc<uint8_t>>;

// A contiguous host tensor: shape, dtype and little-endian bytes — the data
// model of sapient_core::Tensor (crates/sapient-core/src/tensor.rs:22-29).
// Copies share one byte buffer, as the reference's tensors share one
// refcounted buffer (an Arc, crates/sapient-core/src/buffer.rs:54): passing
// or returning a tensor copies no bytes; bytes_mut() first gives this tensor
// its own bytes when they are shared (copy on write).
class Tensor {
 public:
    Tensor() = default;
    static Tensor from_f32(const std::vector<float>& data, std::vector<size_t> shape);
    // Little-endian f32 bytes, taken without a copy (Tensor::from_f32_vec, tensor.rs:51-71).
    static Tensor from_f32_bytes(Bytes bytes, std::vector<size_t> shape);
    static Tensor from_f16_bytes(Bytes bytes, std::vector<size_t> shape);
    static Tensor from_bf16_bytes(Bytes bytes, std::vector<size_t> shape);
    // Packed GGUF blocks; the byte count must equal byte_count(dt, numel)
    // (tensor.rs:143-169).
    static Tensor from_quant_bytes(Bytes bytes, std::vector<size_t> shape, DType dt);

    const std::vector<size_t>& shape() const { return shape_; }
    DType dtype() const { return dtype_; }
    size_t numel() const;
    const Bytes& bytes() const;
    // The same bytes under another shape of equal numel (Tensor::reshape), shared.
    Tensor reshaped(std::vector<size_t> shape) const;
    // The bytes, writable in place (Tensor::as_bytes_mut, tensor.rs:590); shared bytes are copied first.
    Bytes& bytes_mut();
    // The values of an F32 tensor (as_f32_slice); throws for other dtypes.
    std::vector<float> as_f32() const;

 private:
    friend class HipLlmBackend;  // builds results on shared byte buffers
    Tensor(std::vector<size_t> shape, DType dt, Bytes bytes)
        : shape_(std::move(shape)), dtype_(dt), bytes_(std::make_shared<Bytes>(std::move(bytes))) {}
    Tensor(std::vector<size_t> shape, DType dt, std::shared_ptr<Bytes> bytes)
        : shape_(std::move(shape)), dtype_(dt), bytes_(std::move(bytes)) {}
    std::vector<size_t> shape_;
    DType dtype_ = DType::F32;
    std::shared_ptr<Bytes> bytes_;  // null: no bytes
};

// The op surface of the LlmBackend trait on this path
// (crates/sapient-models/src/forward/backend.rs:57-115) plus the fused
// extensions, which default to compositions of the trait's own ops as the
// Rust default methods do. HipLlmBackend implements it; a caller may hand
// HipLlmBackend another implementation (its CPU backend) for the debug
// switches below.
class LlmBackend {
 public:
    virtual ~LlmBackend() = default;
    virtual const char* name() const = 0;

    // LlmBackend::rms_norm (backend.rs:72 → layernorm.rs:75-106): f32 output.
    virtual Tensor rms_norm(const Tensor& x, const Tensor& weight, float eps) = 0;
    // LlmBackend::layer_norm (backend.rs:73-79 → layernorm.rs:17-69, last axis):
    // `bias` may be null; f32 output.
    virtual Tensor layer_norm(const Tensor& x, const Tensor& weight, const Tensor* bias, float eps) = 0;
    // common::add_bias_last_dim (common.rs:556-569), the bias step of
    // LlmBackend::linear_3d_bias (backend.rs:64-70): y F32, bias [y.last_dim].
    virtual Tensor add_bias_last_dim(const Tensor& y, const Tensor& bias) = 0;
    // LlmBackend::silu / gelu (elementwise.rs:141-143, :120-127): F32 input only.
    virtual Tensor silu(const Tensor& x) = 0;
    virtual Tensor gelu(const Tensor& x) = 0;
    // elementwise::gelu_erf (elementwise.rs:135-138): F32 input only.
    virtual Tensor gelu_erf(const Tensor& x) = 0;
    // LlmBackend::add / mul (elementwise.rs:27-69): same length or a length-1 side.
    virtual Tensor add(const Tensor& a, const Tensor& b) = 0;
    virtual Tensor mul(const Tensor& a, const Tensor& b) = 0;
    // LlmBackend::apply_rope_positions (rope.rs:18-62): x [B, H, S, D].
    virtual Tensor apply_rope_positions(const Tensor& x, const std::vector<size_t>& positions, float base) = 0;
    // LlmBackend::apply_rope_partial (rope.rs:71-78, :83-136).
    virtual Tensor apply_rope_partial(const Tensor& x, const std::vector<size_t>& positions, float base,
                                      size_t rotary_dim) = 0;
    // RoPE on adjacent pairs (x[2i], x[2i+1]) — the layout of GGUF's unpermuted
    // q/k rows (gguf_weights.rs:113-115).
    virtual Tensor apply_rope_interleaved(const Tensor& x, const std::vector<size_t>& positions, float base) = 0;
    // common::embed_tokens (common.rs:164-179): weight [vocab, hidden] →
    // [1, ids.size(), hidden] f32; an id >= vocab is an error.
    virtual Tensor embed_tokens(const Tensor& weight, const std::vector<uint32_t>& ids) = 0;

    // Fused extensions: (rms_norm(residual + x), residual + x) and silu(gate) · up.
    virtual std::pair<Tensor, Tensor> add_rms_norm(const Tensor& x, const Tensor& residual, const Tensor& weight,
                                                   float eps) {
        Tensor r = add(residual, x);
        Tensor y = rms_norm(r, weight, eps);
        return {std::move(y), std::move(r)};
    }
    virtual Tensor swiglu(const Tensor& gate, const Tensor& up) { return mul(silu(gate), up); }
};

// Debug switches, read from the environment when a HipLlmBackend is built —
// the HIP counterparts of SAPIENT_MLX_DISABLE / SAPIENT_MLX_VERIFY
// (backend.rs:191-216):
//   SAPIENT_HIP_DISABLE=rms_norm,rope,…  routes the listed ops ("all": every op)
//     to the backend given to the constructor, so a wrong-numbers kernel can be
//     found per op without rebuilding. Op names: rms_norm, layer_norm, add_bias,
//     silu, gelu, gelu_erf, add, mul, rope (all three RoPE methods),
//     add_rms_norm, swiglu, embed. With no backend given, a disabled op raises
//     Error; nothing falls back silently.
//   SAPIENT_HIP_VERIFY=1  runs the given backend beside the first 64 HIP calls
//     and prints "[hip-verify] <op> #<n> max_abs_diff=… cpu_rms=…" to stderr;
//     the HIP result is returned.
// Unlike the Metal backend, a failed HIP call is never retried on the CPU.
class HipLlmBackend final : public LlmBackend {
 public:
    // Binds the current HIP device and creates one stream (default priority).
    // `cpu`, if given, must outlive this backend; only the debug switches use it.
    explicit HipLlmBackend(LlmBackend* cpu = nullptr);
    ~HipLlmBackend() override;
    HipLlmBackend(const HipLlmBackend&) = delete;
    HipLlmBackend& operator=(const HipLlmBackend&) = delete;

    // A gfx950 device is present and the library answers.
    static bool is_available();
    const char* name() const override { return "hip"; }

    Tensor rms_norm(const Tensor& x, const Tensor& weight, float eps) override;
    // kernels::layernorm::rms_norm with the kernel's optional weight (graph path).
    Tensor rms_norm(const Tensor& x, const Tensor* weight, float eps);
    Tensor layer_norm(const Tensor& x, const Tensor& weight, const Tensor* bias, float eps) override;
    // kernels::layernorm::layer_norm over the axes from `axis` on; weight and bias optional.
    Tensor layer_norm(const Tensor& x, const Tensor* weight, const Tensor* bias, int64_t axis, float eps);
    Tensor add_bias_last_dim(const Tensor& y, const Tensor& bias) override;
    Tensor silu(const Tensor& x) override;
    Tensor gelu(const Tensor& x) override;
    Tensor gelu_erf(const Tensor& x) override;
    Tensor add(const Tensor& a, const Tensor& b) override;
    Tensor mul(const Tensor& a, const Tensor& b) override;
    Tensor apply_rope_positions(const Tensor& x, const std::vector<size_t>& positions, float base) override;
    Tensor apply_rope_partial(const Tensor& x, const std::vector<size_t>& positions, float base,
                              size_t rotary_dim) override;
    Tensor apply_rope_interleaved(const Tensor& x, const std::vector<size_t>& positions, float base) override;
    Tensor embed_tokens(const Tensor& weight, const std::vector<uint32_t>& ids) override;
    // One fused kernel each (sph_add_rms_norm, sph_swiglu).
    std::pair<Tensor, Tensor> add_rms_norm(const Tensor& x, const Tensor& residual, const Tensor& weight,
                                           float eps) override;
    Tensor swiglu(const Tensor& gate, const Tensor& up) override;

    // common::update_kv_cache / update_kv_cache_q8 (crates/sapient-models/src/forward/common.rs:355-434,
    // :449-528), the trait path's cache update (llama.rs:489-490): new_k [b, h, new_seq, hd] (any float
    // dtype) is appended after the current_seq_len valid rows of cache [b, h, max_seq, hd] (F32, or
    // Q8_0 blocks), sliding the window once the cache is full; the cache's bytes are updated and the
    // live prefix is returned as F32 [b, h, min(current_seq_len + new_seq, max_seq), hd] (the view the
    // F32 path returns, the dequantized copy the Q8_0 path returns). Errors as the reference's
    // ("update_kv_cache expects 4-D tensors", "update_kv_cache shape mismatch", "new tokens … exceeds
    // max cache size …", and "Tensor dtype is not F32" for an F16 / BF16 cache, tensor.rs:599-602).
    Tensor update_kv_cache(Tensor& cache, size_t current_seq_len, const Tensor& new_k);

    // RoPE reads its angles from a table of positions 0 .. rows - 1 kept per (base, rotary_dim):
    // the reference's rope_cos_sin_cache (crates/sapient-backends/cpu/src/kernels/rope.rs:140-153),
    // evaluated on the host with the libm the reference calls (sph_rope_table), held on the device
    // and grown (doubling) when a call reaches a later position. Calls with a position at or past
    // this many rows evaluate sin/cos on the device instead (sph_rope).
    static constexpr size_t kRopeTableMaxRows = size_t(1) << 18;

    // The switches as read at construction.
    bool disabled(const char* op) const;
    bool verifying() const { return verify_; }

 private:
    // A device allocation owned by one call; freed on scope exit (also when a
    // later upload throws), or earlier by release().
    struct DeviceBuf {
        void* ptr = nullptr;
        size_t bytes = 0;
        DeviceBuf() = default;
        DeviceBuf(const DeviceBuf&) = delete;
        DeviceBuf& operator=(const DeviceBuf&) = delete;
        DeviceBuf(DeviceBuf&& o) noexcept : ptr(o.ptr), bytes(o.bytes) { o.ptr = nullptr; }
        DeviceBuf& operator=(DeviceBuf&&) = delete;
        ~DeviceBuf();
    };
    DeviceBuf upload(const void* host, size_t bytes);
    DeviceBuf alloc(size_t bytes);
    void release(DeviceBuf& b);
    void download(const DeviceBuf& b, void* host, size_t bytes);
    // One call's host operands as device addresses: page-locked tensor bytes in place, small ones
    // through page-locked staging, others through device buffers.
    class Operands;
    // Page-locked staging for a call's small operands, which the kernels read and write in place:
    // chunks kept for the backend's lifetime and reused by every call (calls hold mu_ and wait for
    // their work). stage() returns a slot of `bytes` (host and device addresses; null when no
    // page-locked memory could be had); stage_reset() frees every slot.
    struct StageSlot {
        void* host;
        void* dev;
    };
    struct StageChunk {
        void* host;
        void* dev;
        size_t cap;
    };
    StageSlot stage(size_t bytes);
    void stage_reset() { stage_chunk_ = stage_used_ = 0; }
    std::vector<StageChunk> stage_chunks_;
    size_t stage_chunk_ = 0, stage_used_ = 0;  // the chunk being filled, and its bytes handed out
    // Uninitialised host bytes for a result of n bytes (every result writes all of them); large
    // ones are page-locked blocks freed by dropped tensors, pages already mapped, when one fits.
    static std::shared_ptr<Bytes> result_bytes(size_t n);
    Tensor f32_result(std::shared_ptr<Bytes> bytes, std::vector<size_t> shape) const;
    Tensor f32_input(const Tensor& t) const;  // exact widening of f16/bf16 (tensor.rs:331-361)
    Tensor binary(const Tensor& a, const Tensor& b, bool mul);
    Tensor unary_f32(const Tensor& x, const char* op);
    Tensor rope(const Tensor& x, const std::vector<size_t>& positions, float base, size_t rotary_dim, int layout,
                bool partial);
    void check(int status, const char* op) const;
    // The debug switches around one trait op: `hip` computes on the device,
    // `ref` on the given backend.
    template <typename R, typename Hip, typename Ref>
    R routed(const char* op, Hip&& hip, Ref&& ref);
    void report(const char* op, int n, const Tensor& hip, const Tensor& ref);
    void report(const char* op, int n, const std::pair<Tensor, Tensor>& hip, const std::pair<Tensor, Tensor>& ref);
    // The device paths of the fused, bias and embedding ops.
    std::pair<Tensor, Tensor> fused_add_rms_norm(const Tensor& x, const Tensor& residual, const Tensor& weight,
                                                 float eps);
    Tensor fused_swiglu(const Tensor& gate, const Tensor& up);
    Tensor bias_last_dim(const Tensor& y, const Tensor& bias);
    Tensor gather_rows(const Tensor& weight, const std::vector<uint32_t>& ids);

    // One angle table: `rows` positions of rotary_dim / 2 pairs, cos then sin, on the host and in
    // one device buffer (cos rows, then sin rows).
    struct RopeTable {
        float base = 0.0f;
        size_t rotary_dim = 0;
        size_t rows = 0;
        std::vector<float> cs, sn;
        void* dev = nullptr;
    };
    // The table for (base, rotary_dim) holding at least `rows` positions; called under mu_.
    const RopeTable& rope_table(float base, size_t rotary_dim, size_t rows);
    std::vector<std::unique_ptr<RopeTable>> rope_tables_;

    void* stream_ = nullptr;
    std::mutex mu_;
    LlmBackend* cpu_ = nullptr;
    std::vector<std::string> disabled_;
    bool verify_ = false;
    int verified_ = 0;  // calls cross-checked so far (under verify_mu_)
    std::mutex verify_mu_;
};

// Graph-side ops the HIP backend executes: the ExecutionBackend's supports_op
// set of the path (crates/sapient-backends/cpu/src/backend.rs:168-196 lists
// the CPU's); every other op stays on the CPU backend.
enum class OpKind { Add, Mul, Silu, Gelu, RmsNorm, LayerNorm, RotaryEmbedding, Embedding };

// The attributes these ops carry in OpType (epsilon, axis, base).
struct OpAttrs {
    float epsilon = 1e-5f;
    int64_t axis = -1;
    float base = 10000.0f;
};

// The per-node part of ExecutionBackend::execute for the path: one arm of
// CpuBackend::dispatch (cpu/src/backend.rs:239-487) per OpKind, with its input
// order (nullptr for an absent optional input) and output shapes. Walking the
// graph stays with the caller's executor. Differences from the CPU arms: an
// embedding id >= vocab is an error here (the CPU arm indexes out of bounds).
class HipExecutionBackend {
 public:
    explicit HipExecutionBackend(HipLlmBackend& llm) : llm_(llm) {}
    const char* name() const { return "hip"; }
    static bool supports_op(OpKind op);
    std::vector<Tensor> dispatch(OpKind op, const OpAttrs& attrs, const std::vector<const Tensor*>& inputs);

 private:
    HipLlmBackend& llm_;
};

}  // namespace sapient_hip
