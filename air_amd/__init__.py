"""air_amd -- AIR's quantized linear engine, MI355X-native.

The product is ``libair_hip.so`` (HIP kernels for gfx950 behind the C ABI of
include/air_hip.h) and ``libair_host.so`` (the C++20 executor contract:
execution plans, capability validation, the HIP prepared model and the
capacity / micro-batch schedulers).  This Python package only locates and
binds those libraries; it performs no computation of its own.
"""
from . import capi  # noqa: F401

__all__ = ["capi"]
