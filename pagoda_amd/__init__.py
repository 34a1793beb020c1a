"""pagoda_amd — MI355X (gfx950) decode backend for pagoda.

The compute lives in libpagoda_hip.so (hand-written HIP kernels behind the C
ABI of include/pagoda_hip.h). This package is the Python host mirror used by
tests and the bench: device selection by PAGODA_DEVICE, quantized matrices,
and the model/session surface of the reference's ModelEngine/ModelSession
(pagoda/src/model.rs:66-195).
"""
from ._lib import LIB_PATH, PagodaError, lib  # noqa: F401
from .device import Device, Event, device_from_env  # noqa: F401
from .matrix import Matrix  # noqa: F401

__all__ = ["LIB_PATH", "PagodaError", "lib", "Device", "device_from_env", "Matrix"]
