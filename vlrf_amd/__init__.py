"""vlrf_amd - MI355X (gfx950) HIP decode backend for VLRF, Python binding.

The product is the native library vlrf_amd/libvlrf_hip.so (C ABI declared in
include/vlrf_hip.h).  This module binds it with ctypes for tests and the
benchmark; it has no CPU fallback: every call runs the HIP kernels, and
importing it without a built library raises.
"""
from ._lib import (HipError, lib, check, DT_F32, DT_Q4_0, DT_Q8_0, KV_F32, KV_F16, KV_Q8_0,  # noqa: F401
                   LIB_PATH)
from .runtime import Context, DeviceBuffer, KVCache, QuantWeight, Model  # noqa: F401
from . import formats  # noqa: F401
