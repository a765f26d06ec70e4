// abi.cpp — library identity and status strings for the C ABI.
#include "sapient_hip.h"

extern "C" int sph_abi_version(void) { return SPH_ABI_VERSION; }

extern "C" const char* sph_status_string(int status) {
    switch (status) {
    case SPH_OK: return "ok";
    case SPH_EINVAL: return "invalid argument (null pointer, dtype, shape or alignment)";
    case SPH_EHIP: return "HIP runtime error while enqueueing work";
    case SPH_ERANGE: return "token id out of vocab range";
    case SPH_ENODEV: return "no usable gfx950 device";
    default: return "unknown status";
    }
}
