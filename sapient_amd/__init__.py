"""sapient_amd — MI355X (gfx950) HIP kernels for sapient's fused per-layer op set.

The product is ``libsapient_hip.so`` (C ABI: ``include/sapient_hip.h``); this
package builds it (:mod:`sapient_amd.build`), binds it (:mod:`sapient_amd._lib`)
and exposes device-resident calls on torch tensors (:mod:`sapient_amd.ops`).
"""
from ._lib import (BF16, F16, F32, Q4_K, Q6_K, Q8_0, LIB_PATH, SapientHipError, lib)

__all__ = ["lib", "LIB_PATH", "SapientHipError", "F32", "F16", "BF16", "Q8_0", "Q4_K", "Q6_K"]
