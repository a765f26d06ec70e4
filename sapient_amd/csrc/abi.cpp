// abi.cpp — library identity and status strings for the C ABI, and the
// per-device facts the launchers size their grids by.
#include <atomic>

#include "sph_common.h"

extern "C" int sph_abi_version(void) { return SPH_ABI_VERSION; }

extern "C" const char* sph_status_string(int status) {
    switch (status) {
    case SPH_OK: return "ok";
    case SPH_EINVAL: return "invalid argument (null pointer, dtype, shape or alignment)";
    case SPH_EHIP: return "HIP runtime error while enqueueing work";
    case SPH_ERANGE: return "index out of range (token id >= vocab, or cache positions past max_seq)";
    case SPH_ENODEV: return "no usable gfx950 device";
    case SPH_ESTATE: return "one-time device set-up cannot run while the stream is being captured (call sph_init first)";
    default: return "unknown status";
    }
}

namespace sph {

int device_cu_count() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cache[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace sph
