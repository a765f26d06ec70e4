// hip_llm_backend.cpp — the C++ host-side mirror of sapient's LlmBackend op
// surface (crates/sapient-models/src/forward/backend.rs:57-115) over the C ABI.
//
// Each op runs the HIP kernels on this backend's stream over its host inputs,
// waits, and returns a new host tensor — the round trip the reference's MLX
// backend makes per op (backend.rs:520-600). Tensor bytes of 1 MiB or more are
// page-locked host memory, which the kernels read and write in place through
// its device mapping (both directions of the host link at once, and a gather
// reads only the table rows it needs); smaller operands are copied through
// page-locked staging. No tensor is cached on the device between calls (only
// the RoPE angle tables, which depend on nothing but (base, rotary_dim)): a host
// tensor's address can be reused once it is freed, so caching by pointer (as
// the MLX backend does, backend.rs:483-508, where Arc lifetimes make it safe)
// would risk a stale copy. Output dtypes, validation and error messages follow
// the reference's CPU kernels.
#include "sapient_hip_backend.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <unordered_map>

namespace sapient_hip {

const char* dtype_name(DType dt) {
    switch (dt) {
    case DType::F32: return "f32";
    case DType::F16: return "f16";
    case DType::BF16: return "bf16";
    case DType::Q4_0: return "q4_0";
    case DType::Q8_0: return "q8_0";
    case DType::Q4_K: return "q4_k";
    case DType::Q5_K: return "q5_k";
    case DType::Q6_K: return "q6_k";
    }
    return "?";
}

bool is_quantized(DType dt) {
    return dt == DType::Q4_0 || dt == DType::Q8_0 || dt == DType::Q4_K || dt == DType::Q5_K || dt == DType::Q6_K;
}

size_t byte_count(DType dt, size_t numel) {
    switch (dt) {
    case DType::F32: return numel * 4;
    case DType::F16:
    case DType::BF16: return numel * 2;
    case DType::Q4_0: return numel / 32 * 18;
    case DType::Q8_0: return numel / 32 * 34;
    case DType::Q4_K: return numel / 256 * 144;
    case DType::Q5_K: return numel / 256 * 176;
    case DType::Q6_K: return numel / 256 * 210;
    }
    return 0;
}

static size_t product(const std::vector<size_t>& s) {
    size_t n = 1;
    for (size_t d : s) n *= d;
    return n;
}

static std::string shape_str(const std::vector<size_t>& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

// ─────────────────────────────── Tensor ───────────────────────────────
size_t Tensor::numel() const { return product(shape_); }

Tensor Tensor::from_f32(const std::vector<float>& data, std::vector<size_t> shape) {
    if (product(shape) != data.size())
        throw Error("shape mismatch: expected " + std::to_string(product(shape)) + " elements, got " +
                    std::to_string(data.size()));
    Bytes b(data.size() * 4);
    if (!data.empty()) std::memcpy(b.data(), data.data(), b.size());
    return Tensor(std::move(shape), DType::F32, std::move(b));
}

Tensor Tensor::from_f32_bytes(Bytes bytes, std::vector<size_t> shape) {
    if (bytes.size() != product(shape) * 4)
        throw Error("shape mismatch: expected " + std::to_string(product(shape) * 4) + " bytes, got " +
                    std::to_string(bytes.size()));
    return Tensor(std::move(shape), DType::F32, std::move(bytes));
}

const Bytes& Tensor::bytes() const {
    static const Bytes kNone;
    return bytes_ ? *bytes_ : kNone;
}

Bytes& Tensor::bytes_mut() {
    if (!bytes_)
        bytes_ = std::make_shared<Bytes>();
    else if (bytes_.use_count() > 1)
        bytes_ = std::make_shared<Bytes>(*bytes_);
    return *bytes_;
}

Tensor Tensor::from_f16_bytes(Bytes bytes, std::vector<size_t> shape) {
    if (bytes.size() != product(shape) * 2)
        throw Error("shape mismatch: expected " + std::to_string(product(shape) * 2) + " bytes, got " +
                    std::to_string(bytes.size()));
    return Tensor(std::move(shape), DType::F16, std::move(bytes));
}

Tensor Tensor::from_bf16_bytes(Bytes bytes, std::vector<size_t> shape) {
    if (bytes.size() != product(shape) * 2)
        throw Error("shape mismatch: expected " + std::to_string(product(shape) * 2) + " bytes, got " +
                    std::to_string(bytes.size()));
    return Tensor(std::move(shape), DType::BF16, std::move(bytes));
}

Tensor Tensor::from_quant_bytes(Bytes bytes, std::vector<size_t> shape, DType dt) {
    if (!is_quantized(dt))
        throw Error(std::string("type mismatch: expected a quantized dtype (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K), got ") + dtype_name(dt));
    const size_t expected = byte_count(dt, product(shape));
    if (bytes.size() != expected)
        throw Error("shape mismatch: expected " + std::to_string(expected) + " bytes, got " + std::to_string(bytes.size()));
    return Tensor(std::move(shape), dt, std::move(bytes));
}

Tensor Tensor::reshaped(std::vector<size_t> shape) const {
    size_t n = 1;
    for (size_t d : shape) n *= d;
    if (n != numel()) throw Error("cannot reshape " + shape_str(shape_) + " to " + shape_str(shape));
    return Tensor(std::move(shape), dtype_, bytes_);  // shares the bytes
}

std::vector<float> Tensor::as_f32() const {
    if (dtype_ != DType::F32) throw Error(std::string("type mismatch: expected f32, got ") + dtype_name(dtype_));
    std::vector<float> v(numel());
    if (bytes().size() != v.size() * 4) throw Error("tensor holds no f32 data for its shape");
    if (!v.empty()) std::memcpy(v.data(), bytes_->data(), v.size() * 4);
    return v;
}

// ─────────────────────────────── backend ───────────────────────────────
static void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(std::string("hip: ") + what + ": " + hipGetErrorString(e));
}

bool HipLlmBackend::is_available() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return false;
    return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 && sph_abi_version() == SPH_ABI_VERSION;
}

// SAPIENT_HIP_DISABLE: comma-separated, trimmed, lower-cased, empties dropped
// (the parsing of mlx_disabled, backend.rs:194-207).
static std::vector<std::string> disable_list() {
    std::vector<std::string> out;
    const char* v = std::getenv("SAPIENT_HIP_DISABLE");
    if (!v) return out;
    std::string item;
    auto flush = [&] {
        size_t b = 0, e = item.size();
        while (b < e && std::isspace((unsigned char)item[b])) ++b;
        while (e > b && std::isspace((unsigned char)item[e - 1])) --e;
        std::string t = item.substr(b, e - b);
        for (char& c : t) c = (char)std::tolower((unsigned char)c);
        if (!t.empty()) out.push_back(t);
        item.clear();
    };
    for (const char* p = v; *p; ++p) {
        if (*p == ',') flush();
        else item += *p;
    }
    flush();
    return out;
}

// ─────────────────────────── host byte blocks ───────────────────────────
namespace {

constexpr size_t kLargeBlock = size_t(1) << 20;  // page-locked and recycled from this size on
constexpr size_t kMaxHeld = size_t(4) << 30;      // freed bytes kept for reuse, at most

// Large host blocks: handed out, and freed ones kept (by size) for the next request needing between
// half and all of one. Process-wide, and never destroyed: tensors may outlive every backend, and
// blocks still held at exit go back to the system with the process.
class HostBlocks {
 public:
    void* take(size_t n) {
        {
            std::lock_guard<std::mutex> lock(mu_);
            auto it = free_.lower_bound(n);
            if (it != free_.end() && it->first / 2 <= n) {
                it = std::prev(free_.upper_bound(it->first));  // the most recently freed of that size
                const Block b = it->second;
                held_ -= it->first;
                free_.erase(it);
                live_.emplace(b.ptr, b);
                return b.ptr;
            }
        }
        Block b{nullptr, n, false, nullptr};
        // Portable: mapped for every device, whichever is current when a kernel reads it.
        if (pinnable() && hipHostMalloc(&b.ptr, n, hipHostMallocPortable) == hipSuccess && b.ptr != nullptr) {
            b.pinned = true;
            if (hipHostGetDevicePointer(&b.dev, b.ptr, 0) != hipSuccess) {
                b.dev = nullptr;  // usable for transfers, not in place
                (void)hipGetLastError();
            }
        } else {
            (void)hipGetLastError();  // a refused page-locked allocation falls back to the heap
            b.ptr = ::operator new(n);
        }
        try {
            std::lock_guard<std::mutex> lock(mu_);
            live_.emplace(b.ptr, b);
        } catch (...) {
            release(b);
            throw;
        }
        return b.ptr;
    }

    // The device address of n bytes from p when they lie in one page-locked block handed out here
    // (p its start), else null.
    void* device_view(const void* p, size_t n) {
        std::lock_guard<std::mutex> lock(mu_);
        auto it = live_.find(const_cast<void*>(p));
        if (it == live_.end() || !it->second.pinned || n > it->second.size) return nullptr;
        return it->second.dev;
    }

    void give(void* p) noexcept {
        Block b{};
        {
            std::lock_guard<std::mutex> lock(mu_);
            auto it = live_.find(p);
            if (it == live_.end()) return;  // not handed out here: nothing to do
            b = it->second;
            live_.erase(it);
            if (held_ + b.size <= kMaxHeld) {
                try {
                    free_.emplace(b.size, b);
                    held_ += b.size;
                    return;
                } catch (...) {
                }
            }
        }
        release(b);
    }

 private:
    struct Block {
        void* ptr;
        size_t size;
        bool pinned;
        void* dev;  // the block's address on the device (pinned blocks), or null
    };

    static void release(const Block& b) noexcept {
        if (!b.pinned)
            ::operator delete(b.ptr);
        else if (!exiting())  // at exit the runtime may be gone; the system takes the pages back
            (void)hipHostFree(b.ptr);
    }

    // Set by an exit handler registered after the runtime's set-up (at the first page-locked
    // allocation), so it runs before the runtime's own teardown.
    static std::atomic<bool>& exiting() {
        static std::atomic<bool> flag{false};
        return flag;
    }

    // A HIP device is present (checked once): page-locked memory is only worth its cost then.
    static bool pinnable() {
        static const bool yes = [] {
            int n = 0;
            const bool ok = hipGetDeviceCount(&n) == hipSuccess && n > 0;
            (void)hipGetLastError();
            if (ok) std::atexit([] { exiting().store(true); });
            return ok;
        }();
        return yes;
    }

    std::mutex mu_;
    std::unordered_map<void*, Block> live_;
    std::multimap<size_t, Block> free_;  // by size; equal sizes in the order freed
    size_t held_ = 0;
};

HostBlocks& host_blocks() {
    static HostBlocks* blocks = new HostBlocks;
    return *blocks;
}

}  // namespace

// The device address of a tensor's page-locked bytes, or null for bytes a kernel cannot reach in
// place (heap memory: small tensors, or where page-locked memory was refused).
static void* mapped(const void* p, size_t n) {
    if (p == nullptr || n < kLargeBlock) return nullptr;
    return host_blocks().device_view(p, n);
}

void* host_bytes_alloc(size_t n) {
    if (n < kLargeBlock) return ::operator new(n == 0 ? 1 : n);
    return host_blocks().take(n);
}

void host_bytes_free(void* p, size_t n) noexcept {
    if (p == nullptr) return;
    if (n < kLargeBlock)
        ::operator delete(p);
    else
        host_blocks().give(p);
}

std::shared_ptr<Bytes> HipLlmBackend::result_bytes(size_t n) { return std::make_shared<Bytes>(n); }

Tensor HipLlmBackend::f32_result(std::shared_ptr<Bytes> bytes, std::vector<size_t> shape) const {
    if (bytes->size() != product(shape) * 4)
        throw Error("shape mismatch: expected " + std::to_string(product(shape) * 4) + " bytes, got " +
                    std::to_string(bytes->size()));
    return Tensor(std::move(shape), DType::F32, std::move(bytes));
}

HipLlmBackend::HipLlmBackend(LlmBackend* cpu) : cpu_(cpu) {
    if (!is_available()) throw Error("hip: no gfx950 device available");
    hipStream_t s = nullptr;
    hip_ok(hipStreamCreate(&s), "stream create");  // default priority
    stream_ = s;
    disabled_ = disable_list();
    const char* v = std::getenv("SAPIENT_HIP_VERIFY");
    verify_ = v != nullptr && std::strcmp(v, "1") == 0;
    if (verify_ && cpu_ == nullptr) std::fprintf(stderr, "[hip-verify] no CPU backend given; nothing is cross-checked\n");
}

bool HipLlmBackend::disabled(const char* op) const {
    for (const std::string& s : disabled_)
        if (s == op || s == "all") return true;
    return false;
}

template <typename R, typename Hip, typename Ref>
R HipLlmBackend::routed(const char* op, Hip&& hip, Ref&& ref) {
    if (disabled(op)) {
        if (cpu_ == nullptr)
            throw Error(std::string("hip backend: ") + op + ": disabled by SAPIENT_HIP_DISABLE and no CPU backend was given");
        return ref(*cpu_);
    }
    R out = hip();
    if (verify_ && cpu_ != nullptr) {
        int n;
        {
            std::lock_guard<std::mutex> lock(verify_mu_);
            n = verified_ < 64 ? verified_++ : -1;
        }
        if (n >= 0) report(op, n, out, ref(*cpu_));
    }
    return out;
}

// Largest |hip - ref| (NaN against a number counts as infinite) and ref's RMS.
void HipLlmBackend::report(const char* op, int n, const Tensor& hip, const Tensor& ref) {
    if (hip.shape() != ref.shape()) {
        std::fprintf(stderr, "[hip-verify] %s #%d shape %s vs cpu %s\n", op, n, shape_str(hip.shape()).c_str(),
                     shape_str(ref.shape()).c_str());
        return;
    }
    const std::vector<float> a = f32_input(hip).as_f32(), b = f32_input(ref).as_f32();
    double max_abs = 0.0, norm = 0.0;
    for (size_t i = 0; i < a.size(); ++i) {
        const bool na = std::isnan(a[i]), nb = std::isnan(b[i]);
        const double d = (na || nb) ? (na && nb ? 0.0 : INFINITY) : std::fabs((double)a[i] - (double)b[i]);
        if (d > max_abs) max_abs = d;
        norm += (double)b[i] * (double)b[i];
    }
    const double rms = b.empty() ? 0.0 : std::sqrt(norm / (double)b.size());
    std::fprintf(stderr, "[hip-verify] %s #%d shape=%s max_abs_diff=%.6g cpu_rms=%.6g\n", op, n,
                 shape_str(hip.shape()).c_str(), max_abs, rms);
}

void HipLlmBackend::report(const char* op, int n, const std::pair<Tensor, Tensor>& hip,
                           const std::pair<Tensor, Tensor>& ref) {
    report(op, n, hip.first, ref.first);
    report(op, n, hip.second, ref.second);
}

HipLlmBackend::~HipLlmBackend() {
    if (stream_) (void)hipStreamSynchronize(static_cast<hipStream_t>(stream_));
    for (auto& t : rope_tables_)
        if (t->dev) (void)hipFree(t->dev);
    for (const StageChunk& c : stage_chunks_) (void)hipHostFree(c.host);
    if (stream_) (void)hipStreamDestroy(static_cast<hipStream_t>(stream_));
}

// Every call ends with a synchronizing download, so no queued work reads a table this replaces.
const HipLlmBackend::RopeTable& HipLlmBackend::rope_table(float base, size_t rotary_dim, size_t rows) {
    RopeTable* t = nullptr;
    for (auto& e : rope_tables_)
        if (e->rotary_dim == rotary_dim && std::memcmp(&e->base, &base, sizeof base) == 0) t = e.get();
    if (t == nullptr) {
        rope_tables_.push_back(std::make_unique<RopeTable>());
        t = rope_tables_.back().get();
        t->base = base;
        t->rotary_dim = rotary_dim;
    }
    if (rows <= t->rows) return *t;
    const size_t half = rotary_dim / 2;
    size_t target = std::max<size_t>(rows, std::max<size_t>(2 * t->rows, 64));
    if (target > kRopeTableMaxRows) target = std::max(rows, kRopeTableMaxRows);
    // Rows t->rows .. target - 1: positions evaluated as the reference does (rope.rs:48-50).
    std::vector<int64_t> pos(target - t->rows);
    for (size_t i = 0; i < pos.size(); ++i) pos[i] = (int64_t)(t->rows + i);
    t->cs.resize(target * half);
    t->sn.resize(target * half);
    check(sph_rope_table(pos.data(), (int64_t)pos.size(), (int64_t)rotary_dim, base, 1.0f, t->cs.data() + t->rows * half,
                         t->sn.data() + t->rows * half),
          "rope (angle table)");
    void* dev = nullptr;
    hip_ok(hipMalloc(&dev, 2 * target * half * sizeof(float)), "malloc");
    hipStream_t s = static_cast<hipStream_t>(stream_);
    const hipError_t e1 = hipMemcpyAsync(dev, t->cs.data(), target * half * 4, hipMemcpyHostToDevice, s);
    const hipError_t e2 = hipMemcpyAsync(static_cast<float*>(dev) + target * half, t->sn.data(), target * half * 4,
                                         hipMemcpyHostToDevice, s);
    const hipError_t e3 = hipStreamSynchronize(s);
    if (e1 != hipSuccess || e2 != hipSuccess || e3 != hipSuccess) {
        (void)hipFree(dev);
        t->cs.resize(t->rows * half);
        t->sn.resize(t->rows * half);
        hip_ok(e1 != hipSuccess ? e1 : e2 != hipSuccess ? e2 : e3, "upload (angle table)");
    }
    if (t->dev) (void)hipFree(t->dev);
    t->dev = dev;
    t->rows = target;
    return *t;
}

void HipLlmBackend::check(int status, const char* op) const {
    if (status != SPH_OK)
        throw Error(std::string("hip backend: ") + op + ": " + sph_status_string(status) + " (" +
                    std::to_string(status) + ")");
}

HipLlmBackend::DeviceBuf HipLlmBackend::alloc(size_t bytes) {
    DeviceBuf b;
    b.bytes = bytes;
    hip_ok(hipMalloc(&b.ptr, bytes ? bytes : 16), "malloc");
    return b;
}

HipLlmBackend::DeviceBuf HipLlmBackend::upload(const void* host, size_t bytes) {
    DeviceBuf b = alloc(bytes);
    if (bytes) hip_ok(hipMemcpyAsync(b.ptr, host, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream_)), "upload");
    return b;
}

void HipLlmBackend::download(const DeviceBuf& b, void* host, size_t bytes) {
    if (bytes) hip_ok(hipMemcpyAsync(host, b.ptr, bytes, hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream_)), "download");
    hip_ok(hipStreamSynchronize(static_cast<hipStream_t>(stream_)), "synchronize");
}

// Page-locked tensor bytes are used where they lie, through their device mapping: the kernels
// then read and write host memory over the host link, both directions at once (on the test
// machine a streaming kernel reading two 256 MiB host tensors and writing two took 11.9 ms, the
// four copies alone 18.8 ms). Other large bytes (where page-locked memory was refused, or host
// vectors) go through device buffers, uploaded before the kernels or downloaded after them; small
// ones through staging (below). run() enqueues the uploads, the kernels and, when the kernels were
// accepted, the downloads on the backend's stream, waits for them, then copies staged results out:
// the host bytes must stay untouched until it returns.
//
// Small operands (up to kStageMax bytes: weights, ids, positions, decode-step rows) are copied on
// the host into the backend's page-locked staging, which the kernels also use in place: a call then
// costs a launch and a wait, with no device allocation or copy engine. On the test machine that
// took decode-size calls from 43-97 to 14-17 µs each (rms_norm of 1 × 4096 f32 host tensors 49 ->
// 15 µs, swiglu of 1 × 14336 97 -> 17 µs).
constexpr size_t kStageMax = size_t(1) << 20;

// One Operands per backend at a time (it hands out the backend's staging from the start): each op
// makes one under the backend's lock, and ends it before making another.
class HipLlmBackend::Operands {
 public:
    explicit Operands(HipLlmBackend& bk) : bk_(bk) { bk_.stage_reset(); }
    ~Operands() { bk_.stage_reset(); }
    Operands(const Operands&) = delete;
    Operands& operator=(const Operands&) = delete;

    // Device address holding `bytes` bytes of host input.
    const void* in(const void* host, size_t bytes) {
        if (void* d = mapped(host, bytes)) return d;
        if (const StageSlot sl = stage_copy(host, bytes); sl.dev) return sl.dev;
        void* d = buffer(bytes);
        if (bytes) ups_.push_back({d, host, bytes});
        return d;
    }
    // Device address of an output whose bytes end up in `host`.
    void* out(void* host, size_t bytes) {
        if (void* d = mapped(host, bytes)) return d;
        if (bytes > 0 && bytes <= kStageMax) {
            const StageSlot sl = bk_.stage(bytes);
            if (sl.dev) {
                fetches_.push_back({host, sl.host, bytes});
                return sl.dev;
            }
        }
        void* d = buffer(bytes);
        if (bytes) downs_.push_back({host, d, bytes});
        return d;
    }
    // A copy of `host_in` that the kernels update in place, ending up in `host_out`.
    void* staged(const void* host_in, void* host_out, size_t bytes) {
        if (const StageSlot sl = stage_copy(host_in, bytes); sl.dev) {
            fetches_.push_back({host_out, sl.host, bytes});
            return sl.dev;
        }
        void* d = buffer(bytes);
        if (bytes) {
            ups_.push_back({d, host_in, bytes});
            downs_.push_back({host_out, d, bytes});
        }
        return d;
    }

    int run(const std::function<int()>& launch) {
        hipStream_t s = static_cast<hipStream_t>(bk_.stream_);
        for (const Copy& u : ups_) hip_ok(hipMemcpyAsync(u.dst, u.src, u.n, hipMemcpyHostToDevice, s), "upload");
        const int st = launch();
        if (st == SPH_OK)
            for (const Copy& d : downs_) hip_ok(hipMemcpyAsync(d.dst, d.src, d.n, hipMemcpyDeviceToHost, s), "download");
        hip_ok(hipStreamSynchronize(s), "synchronize");
        if (st == SPH_OK)
            for (const Copy& f : fetches_) std::memcpy(f.dst, f.src, f.n);
        return st;
    }

 private:
    struct Copy {
        void* dst;
        const void* src;
        size_t n;
    };
    // A staging slot holding a copy of `host`, or a null one when the operand is too large or no
    // staging could be had.
    StageSlot stage_copy(const void* host, size_t bytes) {
        if (bytes == 0 || bytes > kStageMax) return {nullptr, nullptr};
        const StageSlot sl = bk_.stage(bytes);
        if (sl.dev) std::memcpy(sl.host, host, bytes);
        return sl;
    }
    void* buffer(size_t bytes) {
        bufs_.push_back(bk_.alloc(bytes));
        return bufs_.back().ptr;
    }
    HipLlmBackend& bk_;
    std::vector<DeviceBuf> bufs_;  // freed with the call
    std::vector<Copy> ups_, downs_, fetches_;
};

HipLlmBackend::StageSlot HipLlmBackend::stage(size_t bytes) {
    const size_t n = (bytes + 255) / 256 * 256;  // 256-byte aligned slots
    while (stage_chunk_ < stage_chunks_.size()) {
        StageChunk& c = stage_chunks_[stage_chunk_];
        if (stage_used_ + n <= c.cap) {
            const StageSlot s{static_cast<char*>(c.host) + stage_used_, static_cast<char*>(c.dev) + stage_used_};
            stage_used_ += n;
            return s;
        }
        ++stage_chunk_;
        stage_used_ = 0;
    }
    StageChunk c{nullptr, nullptr, std::max(n, kStageMax)};
    if (hipHostMalloc(&c.host, c.cap, hipHostMallocPortable) != hipSuccess || c.host == nullptr) {
        (void)hipGetLastError();
        return {nullptr, nullptr};
    }
    if (hipHostGetDevicePointer(&c.dev, c.host, 0) != hipSuccess || c.dev == nullptr) {
        (void)hipGetLastError();
        (void)hipHostFree(c.host);
        return {nullptr, nullptr};
    }
    stage_chunks_.push_back(c);
    stage_chunk_ = stage_chunks_.size() - 1;
    stage_used_ = n;
    return {c.host, c.dev};
}

HipLlmBackend::DeviceBuf::~DeviceBuf() {
    if (ptr) (void)hipFree(ptr);
}

void HipLlmBackend::release(DeviceBuf& b) {
    if (b.ptr) (void)hipFree(b.ptr);
    b.ptr = nullptr;
}

// Tensor::to_f32_cow for the float dtypes (tensor.rs:331-361): exact widening.
Tensor HipLlmBackend::f32_input(const Tensor& t) const {
    if (t.dtype() == DType::F32) return t;
    if (t.dtype() != DType::F16 && t.dtype() != DType::BF16)
        throw Error(std::string("type mismatch: expected a float tensor, got ") + dtype_name(t.dtype()));
    const size_t n = t.numel();
    if (t.bytes().size() != n * 2) throw Error("tensor holds no half-precision data for its shape");
    std::shared_ptr<Bytes> out = result_bytes(n * 4);
    const uint8_t* b = t.bytes().data();
    uint8_t* o = out->data();
    for (size_t i = 0; i < n; ++i) {
        const uint16_t h = (uint16_t)(b[2 * i] | (b[2 * i + 1] << 8));
        uint32_t u;
        if (t.dtype() == DType::BF16) {
            u = (uint32_t)((h & 0x7FFFu) > 0x7F80u ? (h | 0x40u) : h) << 16;
        } else {
            const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
            if (exp == 0x1F) {
                u = sign | 0x7F800000u | (man ? 0x400000u | (man << 13) : 0u);
            } else if (exp == 0) {
                float f = (float)man * 0x1p-24f;
                std::memcpy(&u, &f, 4);
                u |= sign;
            } else {
                u = sign | ((exp + 112u) << 23) | (man << 13);
            }
        }
        std::memcpy(o + 4 * i, &u, 4);
    }
    return f32_result(std::move(out), t.shape());
}

Tensor HipLlmBackend::rms_norm(const Tensor& x, const Tensor& weight_t, float eps) {
    return routed<Tensor>("rms_norm", [&] { return rms_norm(x, &weight_t, eps); },
                          [&](LlmBackend& c) { return c.rms_norm(x, weight_t, eps); });
}

// layernorm::rms_norm (layernorm.rs:75-106): last axis, weight optional.
Tensor HipLlmBackend::rms_norm(const Tensor& x, const Tensor* weight_t, float eps) {
    std::lock_guard<std::mutex> lock(mu_);
    const auto& s = x.shape();
    const size_t dim = s.empty() ? 1 : s.back();
    const size_t rows = dim ? x.numel() / dim : 0;
    if (x.dtype() != DType::F32 && x.dtype() != DType::F16 && x.dtype() != DType::BF16)
        throw Error(std::string("type mismatch: expected a float tensor, got ") + dtype_name(x.dtype()));
    // The device kernel takes an f32 weight or one of x's type (widened exactly on the host otherwise).
    Tensor wt;
    if (weight_t) {
        wt = (weight_t->dtype() == DType::F32 || weight_t->dtype() == x.dtype()) ? *weight_t : f32_input(*weight_t);
        if (wt.numel() != dim)
            throw Error("shape mismatch: weight " + shape_str(wt.shape()) + " for rows of " + std::to_string(dim));
    }
    auto out = result_bytes(x.numel() * 4);
    Operands ops(*this);
    const void* xd = ops.in(x.bytes().data(), x.bytes().size());
    const void* wd = weight_t ? ops.in(wt.bytes().data(), wt.bytes().size()) : nullptr;
    void* od = ops.out(out->data(), out->size());
    const int st = ops.run([&] {
        return sph_rms_norm(xd, (int)x.dtype(), wd, weight_t ? (int)wt.dtype() : SPH_F32, od, SPH_F32, (int64_t)rows,
                            (int64_t)dim, eps, stream_);
    });
    check(st, "rms_norm");
    return f32_result(std::move(out), s);
}

std::pair<Tensor, Tensor> HipLlmBackend::add_rms_norm(const Tensor& x, const Tensor& residual, const Tensor& weight_t,
                                                      float eps) {
    return routed<std::pair<Tensor, Tensor>>("add_rms_norm", [&] { return fused_add_rms_norm(x, residual, weight_t, eps); },
                                             [&](LlmBackend& c) { return c.add_rms_norm(x, residual, weight_t, eps); });
}

std::pair<Tensor, Tensor> HipLlmBackend::fused_add_rms_norm(const Tensor& x, const Tensor& residual,
                                                            const Tensor& weight_t, float eps) {
    const Tensor xf = f32_input(x), rf = f32_input(residual);
    if (xf.shape() != rf.shape())
        throw Error("shape mismatch: " + shape_str(xf.shape()) + " vs " + shape_str(rf.shape()));
    std::lock_guard<std::mutex> lock(mu_);
    const size_t dim = xf.shape().empty() ? 1 : xf.shape().back();
    const size_t rows = dim ? xf.numel() / dim : 0;
    const Tensor wt = weight_t.dtype() == DType::F32 ? weight_t : f32_input(weight_t);
    if (wt.numel() != dim) throw Error("shape mismatch: weight " + shape_str(wt.shape()) + " for rows of " + std::to_string(dim));
    auto normed = result_bytes(xf.numel() * 4);
    auto sum = result_bytes(xf.numel() * 4);
    Operands ops(*this);
    const void* xd = ops.in(xf.bytes().data(), xf.bytes().size());
    const void* rd = ops.in(rf.bytes().data(), rf.bytes().size());
    void* sd = ops.out(sum->data(), sum->size());
    const void* wd = ops.in(wt.bytes().data(), wt.bytes().size());
    void* od = ops.out(normed->data(), normed->size());
    const int st = ops.run([&] {
        return sph_add_rms_norm_to(xd, rd, sd, SPH_F32, wd, SPH_F32, od, SPH_F32, (int64_t)rows, (int64_t)dim, eps,
                                   stream_);
    });
    check(st, "add_rms_norm");
    return {f32_result(std::move(normed), xf.shape()), f32_result(std::move(sum), xf.shape())};
}

// binary_f32 (elementwise.rs:27-57): both sides widened to f32; same length or
// a length-1 side broadcast; anything else is a ShapeMismatch.
Tensor HipLlmBackend::binary(const Tensor& a0, const Tensor& b0, bool mul) {
    const Tensor a = f32_input(a0), b = f32_input(b0);
    const size_t na = a.numel(), nb = b.numel();
    if (!(na == nb || nb == 1 || na == 1))
        throw Error("shape mismatch: expected " + shape_str(a.shape()) + ", got " + shape_str(b.shape()));
    const std::vector<size_t> shape = (na == nb || nb == 1) ? a.shape() : b.shape();
    const size_t n = (na == nb || nb == 1) ? na : nb;
    std::lock_guard<std::mutex> lock(mu_);
    auto out = result_bytes(n * 4);
    Operands ops(*this);
    const void* ad = ops.in(a.bytes().data(), a.bytes().size());
    const void* bd = ops.in(b.bytes().data(), b.bytes().size());
    void* od = ops.out(out->data(), out->size());
    const int st = ops.run([&] {
        return mul ? sph_mul(ad, (int64_t)na, bd, (int64_t)nb, od, SPH_F32, stream_)
                   : sph_add(ad, (int64_t)na, bd, (int64_t)nb, od, SPH_F32, stream_);
    });
    check(st, mul ? "mul" : "add");
    return f32_result(std::move(out), shape);
}

Tensor HipLlmBackend::add(const Tensor& a, const Tensor& b) {
    return routed<Tensor>("add", [&] { return binary(a, b, false); }, [&](LlmBackend& c) { return c.add(a, b); });
}
Tensor HipLlmBackend::mul(const Tensor& a, const Tensor& b) {
    return routed<Tensor>("mul", [&] { return binary(a, b, true); }, [&](LlmBackend& c) { return c.mul(a, b); });
}

// unary_f32 (elementwise.rs:15-24): only F32 input is accepted.
Tensor HipLlmBackend::unary_f32(const Tensor& x, const char* op) {
    if (x.dtype() != DType::F32) throw Error(std::string("type mismatch: expected f32, got ") + dtype_name(x.dtype()));
    std::lock_guard<std::mutex> lock(mu_);
    auto out = result_bytes(x.numel() * 4);
    Operands ops(*this);
    const void* xd = ops.in(x.bytes().data(), x.bytes().size());
    void* od = ops.out(out->data(), out->size());
    const int64_t n = (int64_t)x.numel();
    const int st = ops.run([&] {
        if (std::strcmp(op, "silu") == 0) return sph_silu(xd, od, SPH_F32, n, stream_);
        if (std::strcmp(op, "gelu_erf") == 0) return sph_gelu_erf(xd, od, SPH_F32, n, stream_);
        return sph_gelu_tanh(xd, od, SPH_F32, n, stream_);
    });
    check(st, op);
    return f32_result(std::move(out), x.shape());
}

Tensor HipLlmBackend::silu(const Tensor& x) {
    return routed<Tensor>("silu", [&] { return unary_f32(x, "silu"); }, [&](LlmBackend& c) { return c.silu(x); });
}
Tensor HipLlmBackend::gelu(const Tensor& x) {
    return routed<Tensor>("gelu", [&] { return unary_f32(x, "gelu"); }, [&](LlmBackend& c) { return c.gelu(x); });
}
Tensor HipLlmBackend::gelu_erf(const Tensor& x) {
    return routed<Tensor>("gelu_erf", [&] { return unary_f32(x, "gelu_erf"); },
                          [&](LlmBackend& c) { return c.gelu_erf(x); });
}

Tensor HipLlmBackend::layer_norm(const Tensor& x, const Tensor& weight, const Tensor* bias, float eps) {
    return routed<Tensor>("layer_norm", [&] { return layer_norm(x, &weight, bias, -1, eps); },
                          [&](LlmBackend& c) { return c.layer_norm(x, weight, bias, eps); });
}

// layernorm::layer_norm (layernorm.rs:17-69): normalises over the axes from
// `axis` on (negative counts from the end); x, weight and bias are widened to
// f32 (to_f32_cow) and the output is f32. Weight and bias are optional.
Tensor HipLlmBackend::layer_norm(const Tensor& x0, const Tensor* weight0, const Tensor* bias0, int64_t axis,
                                 float eps) {
    const Tensor x = f32_input(x0);
    const Tensor w = weight0 ? f32_input(*weight0) : Tensor();
    const Tensor b = bias0 ? f32_input(*bias0) : Tensor();
    const auto& s = x.shape();
    const int64_t nd = (int64_t)s.size();
    const int64_t ax = axis < 0 ? nd + axis : axis;
    if (ax < 0 || ax > nd) throw Error("axis " + std::to_string(axis) + " out of range for " + shape_str(s));
    size_t dim = 1;
    for (int64_t i = ax; i < nd; ++i) dim *= s[i];
    const size_t rows = dim ? x.numel() / dim : 0;
    if (weight0 && w.numel() != dim)
        throw Error("shape mismatch: weight " + shape_str(w.shape()) + " for rows of " + std::to_string(dim));
    if (bias0 && b.numel() != dim) throw Error("shape mismatch: bias " + shape_str(b.shape()) + " for rows of " + std::to_string(dim));
    std::lock_guard<std::mutex> lock(mu_);
    auto out = result_bytes(x.numel() * 4);
    Operands ops(*this);
    const void* xd = ops.in(x.bytes().data(), x.bytes().size());
    const void* wd = weight0 ? ops.in(w.bytes().data(), w.bytes().size()) : nullptr;
    const void* bd = bias0 ? ops.in(b.bytes().data(), b.bytes().size()) : nullptr;
    void* od = ops.out(out->data(), out->size());
    const int st = ops.run([&] {
        return sph_layer_norm(xd, SPH_F32, wd, bd, SPH_F32, od, SPH_F32, (int64_t)rows, (int64_t)dim, eps, stream_);
    });
    check(st, "layer_norm");
    return f32_result(std::move(out), s);
}

// common::add_bias_last_dim (common.rs:556-569): y is F32, the bias any float
// type of length equal to y's last dimension.
Tensor HipLlmBackend::add_bias_last_dim(const Tensor& y, const Tensor& bias0) {
    return routed<Tensor>("add_bias", [&] { return bias_last_dim(y, bias0); },
                          [&](LlmBackend& c) { return c.add_bias_last_dim(y, bias0); });
}

Tensor HipLlmBackend::bias_last_dim(const Tensor& y, const Tensor& bias0) {
    if (y.shape().empty()) throw Error("empty tensor");
    if (y.dtype() != DType::F32) throw Error(std::string("type mismatch: expected f32, got ") + dtype_name(y.dtype()));
    const size_t n = y.shape().back();
    const Tensor b = (bias0.dtype() == DType::F32 || bias0.dtype() == DType::F16 || bias0.dtype() == DType::BF16)
                         ? bias0 : f32_input(bias0);
    if (b.numel() != n)
        throw Error("bias length " + std::to_string(b.numel()) + " does not match last dim " + std::to_string(n));
    std::lock_guard<std::mutex> lock(mu_);
    auto out = result_bytes(y.numel() * 4);
    Operands ops(*this);
    const void* yd = ops.in(y.bytes().data(), y.bytes().size());
    const void* bd = ops.in(b.bytes().data(), b.bytes().size());
    void* od = ops.out(out->data(), out->size());
    const int st = ops.run([&] {
        return sph_add_bias(yd, bd, (int)b.dtype(), od, SPH_F32, (int64_t)y.numel(), (int64_t)n, stream_);
    });
    check(st, "add_bias_last_dim");
    return f32_result(std::move(out), y.shape());
}

Tensor HipLlmBackend::swiglu(const Tensor& gate, const Tensor& up) {
    return routed<Tensor>("swiglu", [&] { return fused_swiglu(gate, up); },
                          [&](LlmBackend& c) { return c.swiglu(gate, up); });
}

Tensor HipLlmBackend::fused_swiglu(const Tensor& gate, const Tensor& up) {
    if (gate.dtype() != DType::F32 || up.dtype() != DType::F32)
        throw Error(std::string("type mismatch: expected f32, got ") + dtype_name(gate.dtype() != DType::F32 ? gate.dtype() : up.dtype()));
    if (gate.numel() != up.numel())
        throw Error("shape mismatch: expected " + shape_str(gate.shape()) + ", got " + shape_str(up.shape()));
    std::lock_guard<std::mutex> lock(mu_);
    auto out = result_bytes(gate.numel() * 4);
    Operands ops(*this);
    const void* gd = ops.in(gate.bytes().data(), gate.bytes().size());
    const void* ud = ops.in(up.bytes().data(), up.bytes().size());
    void* od = ops.out(out->data(), out->size());
    const int st = ops.run([&] { return sph_swiglu(gd, ud, od, SPH_F32, (int64_t)gate.numel(), stream_); });
    check(st, "swiglu");
    return f32_result(std::move(out), gate.shape());
}

// rope.rs:18-62 / :83-136: x [batch, n_heads, seq_len, head_dim] → new f32 tensor.
Tensor HipLlmBackend::rope(const Tensor& x0, const std::vector<size_t>& positions, float base, size_t rotary_dim,
                           int layout, bool partial) {
    const auto& d = x0.shape();
    if (d.size() != 4) throw Error("rank mismatch: expected 4, got " + std::to_string(d.size()));
    const size_t batch = d[0], n_heads = d[1], seq = d[2], head_dim = d[3];
    if (partial) {
        if (rotary_dim == 0 || rotary_dim > head_dim) throw Error("rotary_dim must be in 1..=head_dim");
        if (rotary_dim % 2 != 0) throw Error("RoPE requires even rotary_dim");
    } else if (head_dim % 2 != 0) {
        throw Error("RoPE requires even head_dim");
    }
    if (positions.size() != seq) throw Error("positions length must match seq_len");
    std::vector<int32_t> pos(seq);
    for (size_t i = 0; i < seq; ++i) {
        if (positions[i] > (size_t)INT32_MAX) throw Error("position out of the supported range (< 2^31)");
        pos[i] = (int32_t)positions[i];
    }
    const Tensor x = f32_input(x0);
    // The angles come from this backend's table of positions 0 .. rows - 1 (the reference's
    // rope_cos_sin_cache, evaluated with its libm: the kernel only reads them), grown to the call's
    // last position; a position past the table's cap takes the device sin/cos path.
    size_t last = 0;
    for (size_t p : positions) last = std::max(last, p);
    const bool table = !positions.empty() && last < kRopeTableMaxRows;
    std::lock_guard<std::mutex> lock(mu_);
    const RopeTable* t = table ? &rope_table(base, rotary_dim, last + 1) : nullptr;
    auto out = result_bytes(x.numel() * 4);
    Operands ops(*this);
    void* xd = ops.staged(x.bytes().data(), out->data(), out->size());  // rotated in place
    const int32_t* pd = static_cast<const int32_t*>(ops.in(pos.data(), pos.size() * 4));
    const int st = ops.run([&] {
        if (table) {
            const float* cs = static_cast<const float*>(t->dev);
            return sph_rope_cached(xd, (int64_t)n_heads, nullptr, 0, SPH_F32, layout, cs, cs + t->rows * (rotary_dim / 2),
                                   (int64_t)t->rows, pd, (int64_t)batch, (int64_t)seq, (int64_t)head_dim,
                                   (int64_t)rotary_dim, nullptr, stream_);
        }
        return sph_rope(xd, (int64_t)n_heads, nullptr, 0, SPH_F32, layout, pd, (int64_t)batch, (int64_t)seq,
                        (int64_t)head_dim, (int64_t)rotary_dim, base, 1.0f, stream_);
    });
    check(st, "rope");
    return f32_result(std::move(out), d);
}

Tensor HipLlmBackend::apply_rope_positions(const Tensor& x, const std::vector<size_t>& positions, float base) {
    const size_t head_dim = x.shape().size() == 4 ? x.shape()[3] : 0;
    return routed<Tensor>("rope", [&] { return rope(x, positions, base, head_dim, SPH_ROPE_NEOX, false); },
                          [&](LlmBackend& c) { return c.apply_rope_positions(x, positions, base); });
}

Tensor HipLlmBackend::apply_rope_partial(const Tensor& x, const std::vector<size_t>& positions, float base,
                                         size_t rotary_dim) {
    return routed<Tensor>("rope", [&] { return rope(x, positions, base, rotary_dim, SPH_ROPE_NEOX, true); },
                          [&](LlmBackend& c) { return c.apply_rope_partial(x, positions, base, rotary_dim); });
}

Tensor HipLlmBackend::apply_rope_interleaved(const Tensor& x, const std::vector<size_t>& positions, float base) {
    const size_t head_dim = x.shape().size() == 4 ? x.shape()[3] : 0;
    return routed<Tensor>("rope", [&] { return rope(x, positions, base, head_dim, SPH_ROPE_INTERLEAVED, false); },
                          [&](LlmBackend& c) { return c.apply_rope_interleaved(x, positions, base); });
}

// common.rs:164-217: every id is checked against vocab before any row is read.
Tensor HipLlmBackend::embed_tokens(const Tensor& w, const std::vector<uint32_t>& ids) {
    return routed<Tensor>("embed", [&] { return gather_rows(w, ids); },
                          [&](LlmBackend& c) { return c.embed_tokens(w, ids); });
}

Tensor HipLlmBackend::gather_rows(const Tensor& w, const std::vector<uint32_t>& ids) {
    const auto& d = w.shape();
    if (d.size() != 2) throw Error("embedding table must be [vocab, hidden], got " + shape_str(d));
    const size_t vocab = d[0], hidden = d[1];
    for (uint32_t id : ids)
        if ((size_t)id >= vocab) throw Error("token id " + std::to_string(id) + " out of vocab range");
    std::lock_guard<std::mutex> lock(mu_);
    auto out = result_bytes(ids.size() * hidden * 4);
    Operands ops(*this);
    const void* td = ops.in(w.bytes().data(), w.bytes().size());  // in place when page-locked: only the rows read cross
    const uint32_t* idd = static_cast<const uint32_t*>(ops.in(ids.data(), ids.size() * 4));
    float* od = static_cast<float*>(ops.out(out->data(), out->size()));
    const int st = ops.run([&] {
        return sph_embed(td, (int)w.dtype(), (int64_t)vocab, (int64_t)hidden, idd, (int64_t)ids.size(), od, nullptr,
                         stream_);
    });
    if (st == SPH_EINVAL) throw Error(std::string("unsupported embedding dtype ") + dtype_name(w.dtype()));
    check(st, "embed_tokens");
    return f32_result(std::move(out), {1, ids.size(), hidden});
}

// common.rs:355-434 / :449-528 over sph_kv_cache_update; the Q8_0 prefix is
// dequantized by the gather kernel (its Q8_0 arm is the reference's
// `q as i8 as f32 * d`, common.rs:518-524), reading the cache rows as a table.
Tensor HipLlmBackend::update_kv_cache(Tensor& cache, size_t current_seq_len, const Tensor& new_k) {
    const auto& cd = cache.shape();
    const auto& nd = new_k.shape();
    if (cd.size() != 4 || nd.size() != 4) throw Error("update_kv_cache expects 4-D tensors");
    if (cd[0] != nd[0] || cd[1] != nd[1] || cd[3] != nd[3]) throw Error("update_kv_cache shape mismatch");
    const size_t b = cd[0], h = cd[1], max_seq = cd[2], hd = cd[3], new_seq = nd[2];
    if (new_seq > max_seq)
        throw Error("new tokens " + std::to_string(new_seq) + " exceeds max cache size " + std::to_string(max_seq));
    const DType cdt = cache.dtype();
    // The reference's float path writes through cache.as_f32_slice_mut() (common.rs:378), which
    // refuses any other dtype (tensor.rs:599-602); only Q8_0 has a path of its own.
    if (cdt != DType::F32 && cdt != DType::Q8_0) throw Error("Tensor dtype is not F32");
    if (current_seq_len > max_seq) throw Error("current length " + std::to_string(current_seq_len) + " exceeds the cache");
    const Tensor src = f32_input(new_k);
    std::lock_guard<std::mutex> lock(mu_);
    // The cache's own bytes (copied first if another tensor shares them), written as the reference
    // writes through as_f32_slice_mut. Page-locked bytes are updated where they lie: an append
    // writes only the new rows; a slide moves the kept rows once into a fresh block, which then
    // becomes the cache's storage. Other caches are copied in and back.
    Bytes& cb = cache.bytes_mut();
    const size_t cbytes = cb.size();
    void* cmap = mapped(cb.data(), cbytes);
    const bool slides = current_seq_len + new_seq > max_seq;
    std::shared_ptr<Bytes> fresh = (cmap && slides) ? result_bytes(cbytes) : nullptr;
    void* fmap = fresh ? mapped(fresh->data(), cbytes) : nullptr;
    if (fresh && !fmap) fresh.reset();  // no page-locked block to slide into: the slide runs in place
    int64_t total = 0;
    int st;
    {
        Operands ops(*this);
        const void* sd = ops.in(src.bytes().data(), src.bytes().size());
        // Not page-locked: the cache is copied in (and, for a slide, the moved rows come back from
        // a second copy).
        void* cd = nullptr;
        void* dst = nullptr;  // where a slide moves the kept rows (null: in place)
        if (cmap) {
            cd = cmap;
            dst = fmap;
        } else if (slides) {
            cd = const_cast<void*>(ops.in(cb.data(), cbytes));
            dst = ops.out(cb.data(), cbytes);
        } else {
            cd = ops.staged(cb.data(), cb.data(), cbytes);
        }
        st = ops.run([&] {
            if (dst == nullptr)
                return sph_kv_cache_update(sd, SPH_F32, cd, (int)cdt, (int64_t)(b * h), (int64_t)new_seq,
                                           (int64_t)hd, (int64_t)max_seq, (int64_t)current_seq_len, &total, stream_);
            return sph_kv_cache_update_into(sd, SPH_F32, cd, dst, (int)cdt, (int64_t)(b * h), (int64_t)new_seq,
                                            (int64_t)hd, (int64_t)max_seq, (int64_t)current_seq_len, &total, stream_);
        });
    }
    check(st, "update_kv_cache");
    if (fresh) cache.bytes_ = std::move(fresh);
    const Bytes& now = cache.bytes();
    const size_t n = (size_t)total;
    if (cdt == DType::Q8_0) {
        // The live prefix dequantized by the gather kernel, the cache rows read as a table.
        std::vector<uint32_t> ids(b * h * n);
        for (size_t r = 0; r < b * h; ++r)
            for (size_t s = 0; s < n; ++s) ids[r * n + s] = (uint32_t)(r * max_seq + s);
        auto out = result_bytes(ids.size() * hd * 4);
        Operands ops(*this);
        const void* td = ops.in(now.data(), now.size());
        const uint32_t* idd = static_cast<const uint32_t*>(ops.in(ids.data(), ids.size() * 4));
        float* od = static_cast<float*>(ops.out(out->data(), out->size()));
        st = ops.run([&] {
            return sph_embed(td, SPH_Q8_0, (int64_t)(b * h * max_seq), (int64_t)hd, idd, (int64_t)ids.size(), od,
                             nullptr, stream_);
        });
        check(st, "update_kv_cache (dequantize)");
        return f32_result(std::move(out), {b, h, n, hd});
    }
    // The live prefix [b, h, n, hd] of the F32 cache, head by head.
    auto out = result_bytes(b * h * n * hd * 4);
    for (size_t r = 0; r < b * h; ++r)
        if (n) std::memcpy(out->data() + r * n * hd * 4, now.data() + r * max_seq * hd * 4, n * hd * 4);
    return f32_result(std::move(out), {b, h, n, hd});
}

// ── graph-side dispatch ─────────────────────────────────────────────────────

bool HipExecutionBackend::supports_op(OpKind) { return true; }  // every kind of OpKind runs here

std::vector<Tensor> HipExecutionBackend::dispatch(OpKind op, const OpAttrs& attrs,
                                                  const std::vector<const Tensor*>& in) {
    auto need = [&](size_t i, const char* what) -> const Tensor& {
        if (i >= in.size() || in[i] == nullptr) throw Error(std::string(what));
        return *in[i];
    };
    auto opt = [&](size_t i) -> const Tensor* { return i < in.size() ? in[i] : nullptr; };
    switch (op) {
    case OpKind::Add: return {llm_.add(need(0, "Add: missing a"), need(1, "Add: missing b"))};
    case OpKind::Mul: return {llm_.mul(need(0, "Mul: missing a"), need(1, "Mul: missing b"))};
    case OpKind::Silu: return {llm_.silu(need(0, "Silu: missing input"))};
    case OpKind::Gelu: return {llm_.gelu(need(0, "Gelu: missing input"))};
    case OpKind::RmsNorm: return {llm_.rms_norm(need(0, "RmsNorm: missing input"), opt(1), attrs.epsilon)};
    case OpKind::LayerNorm:
        return {llm_.layer_norm(need(0, "LayerNorm: missing input"), opt(1), opt(2), attrs.axis, attrs.epsilon)};
    case OpKind::RotaryEmbedding: {
        // positions 0 .. seq_len - 1, seq_len = dims[2] (cpu/src/backend.rs:480-487)
        const Tensor& x = need(0, "RoPE: missing input");
        const size_t seq = x.shape().size() > 2 ? x.shape()[2] : 1;
        std::vector<size_t> pos(seq);
        for (size_t i = 0; i < seq; ++i) pos[i] = i;
        return {llm_.apply_rope_positions(x, pos, attrs.base)};
    }
    case OpKind::Embedding: {
        // weight [vocab, hidden] at inputs[0], ids at inputs[1]: F32 values cast to u32
        // (Rust `as`: saturating, NaN → 0) or raw little-endian u32 (cpu/src/backend.rs:381-411)
        const Tensor& w = need(0, "Embedding: missing weight");
        const Tensor& ids_t = need(1, "Embedding: missing input_ids");
        std::vector<uint32_t> ids;
        if (ids_t.dtype() == DType::F32) {
            for (float v : ids_t.as_f32())
                ids.push_back(!(v > 0.0f) ? 0u : (v >= 4294967295.0f ? 0xFFFFFFFFu : (uint32_t)v));
        } else {
            const auto& b = ids_t.bytes();
            for (size_t i = 0; i + 4 <= b.size(); i += 4)
                ids.push_back((uint32_t)b[i] | ((uint32_t)b[i + 1] << 8) | ((uint32_t)b[i + 2] << 16) |
                              ((uint32_t)b[i + 3] << 24));
        }
        const auto& d = ids_t.shape();
        const size_t batch = d.size() >= 2 ? d[0] : 1;
        const size_t seq = d.size() >= 2 ? d[1] : ids.size();
        Tensor out = llm_.embed_tokens(w, ids);
        if (batch * seq != ids.size()) throw Error("Embedding: ids shape " + shape_str(d) + " is not [batch, seq]");
        return {out.reshaped({batch, seq, w.shape()[1]})};
    }
    }
    throw Error("unsupported op");
}

}  // namespace sapient_hip
