"""Device handle: the PAGODA_DEVICE=hip branch of CandleModel::device_from_env
(pagoda-hf/src/lib.rs:409-426)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import call, lib


class Device:
    """One HIP device and the stream every backend call on it is queued on."""

    def __init__(self, spec: str = "hip"):
        h = C.c_void_p()
        call("pgd_device_open", spec.encode(), C.byref(h))
        self.handle = h
        self.spec = spec

    def close(self) -> None:
        if self.handle:
            call("pgd_device_close", self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return int(lib().pgd_device_stream(self.handle) or 0)

    def sync(self) -> None:
        call("pgd_device_sync", self.handle)

    # --- raw device buffers (tests use them without torch) ---
    def alloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        call("pgd_device_malloc", self.handle, C.c_size_t(nbytes), C.byref(p))
        return int(p.value)

    def free(self, ptr: int) -> None:
        call("pgd_device_free", self.handle, C.c_void_p(ptr))

    def upload(self, arr: np.ndarray) -> int:
        arr = np.ascontiguousarray(arr)
        p = self.alloc(arr.nbytes)
        call("pgd_device_memcpy", self.handle, C.c_void_p(p), arr.ctypes.data_as(C.c_void_p), C.c_size_t(arr.nbytes), 0)
        return p

    def download(self, ptr: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        call("pgd_device_memcpy", self.handle, out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), C.c_size_t(out.nbytes), 1)
        return out


class Event:
    """HIP event recorded on the device handle's stream."""

    def __init__(self, dev: Device):
        self.dev = dev
        h = C.c_void_p()
        call("pgd_event_new", dev.handle, C.byref(h))
        self.handle = h

    def record(self) -> "Event":
        call("pgd_event_record", self.handle)
        return self

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        call("pgd_event_elapsed_ms", self.handle, end.handle, C.byref(ms))
        return float(ms.value)

    def __del__(self):
        try:
            call("pgd_event_free", self.handle)
        except Exception:
            pass


def device_from_env() -> Device:
    """PAGODA_DEVICE must be `hip` or `hip:N`; anything else is an error (no
    silent CPU fallback, as in the reference's device_from_env)."""
    spec = os.environ.get("PAGODA_DEVICE", "hip")
    if spec != "hip" and not spec.startswith("hip:"):
        raise ValueError(f"unknown PAGODA_DEVICE {spec!r} for the HIP backend (want hip or hip:N)")
    return Device(spec)
