"""objeta_amd — MI355X (gfx950) selected-expert MoE decode path behind a C ABI.

The compute lives in libobjeta_hip.so (objeta_amd/csrc, include/objeta_hip.h);
this package is the Python mirror of the reference API used by tests and the
benchmark.
"""
from .api import (DeviceBuffer, ExpertCache, ExpertCacheKey, ExpertTable, ExpertTensorKind, HipBackend,
                  HipBackendBuilder, HipError, HostExpertSet, MoeExecutor, PinnedHostBuffer, QGemvShape, QuantBackend, QuantFormat, check,
                  discover_devices)

__all__ = ["DeviceBuffer", "ExpertCache", "ExpertCacheKey", "ExpertTable", "ExpertTensorKind", "HipBackend",
           "HipBackendBuilder", "HipError", "HostExpertSet", "MoeExecutor", "PinnedHostBuffer", "QGemvShape", "QuantBackend", "QuantFormat", "check",
           "discover_devices"]
