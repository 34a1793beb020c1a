"""Quantized matrix handle (QuantMatrix, pagoda-hf/src/qwen3_gemv.rs:640-760)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import call
from .device import Device

FMT_A8, FMT_Q4K, FMT_Q6K, FMT_Q8_0, FMT_Q5_0 = 0, 1, 2, 3, 4
FMT_NAMES = {FMT_A8: "a8", FMT_Q4K: "q4k", FMT_Q6K: "q6k", FMT_Q8_0: "q8_0", FMT_Q5_0: "q5_0"}


def _ptr(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


def act_bytes(nrows: int, k: int) -> int:
    from ._lib import lib

    return int(lib().pgd_act_bytes(nrows, k))


def act_prep_dev(dev: Device, x_ptr: int, ldx: int, nrows: int, k: int, act_ptr: int) -> None:
    call("pgd_act_prep_dev", dev.handle, C.c_void_p(x_ptr), ldx, nrows, k, C.c_void_p(act_ptr))


class Matrix:
    def __init__(self, dev: Device, handle: C.c_void_p):
        self.dev = dev
        self.handle = handle
        fmt, n_out, n_in = C.c_int(), C.c_int(), C.c_int()
        dbytes, abytes = C.c_size_t(), C.c_double()
        call("pgd_matrix_info", handle, C.byref(fmt), C.byref(n_out), C.byref(n_in), C.byref(dbytes), C.byref(abytes))
        self.fmt, self.n_out, self.n_in = fmt.value, n_out.value, n_in.value
        self.dev_bytes, self.algo_bytes = dbytes.value, abytes.value

    # ---- constructors ----
    @classmethod
    def upload_a8(cls, dev: Device, packed: np.ndarray, scales: np.ndarray, biases: np.ndarray, n_out: int, n_in: int):
        packed = np.ascontiguousarray(packed, np.uint32)
        scales = np.ascontiguousarray(scales, np.uint16)
        biases = np.ascontiguousarray(biases, np.uint16)
        assert packed.size == n_out * n_in // 4 and scales.size == biases.size == n_out * (n_in // 64)
        h = C.c_void_p()
        call("pgd_matrix_upload_a8", dev.handle, _ptr(packed), _ptr(scales), _ptr(biases), n_out, n_in, C.byref(h))
        return cls(dev, h)

    @classmethod
    def upload_kq(cls, dev: Device, fmt: int, blocks: np.ndarray, n_out: int, n_in: int):
        """GGML blocks, row-major: Q4_K / Q6_K super-blocks or Q8_0 / Q5_0 blocks."""
        blocks = np.ascontiguousarray(blocks, np.uint8)
        if fmt in (FMT_Q8_0, FMT_Q5_0):
            assert blocks.size == n_out * (n_in // 32) * (34 if fmt == FMT_Q8_0 else 22)
        else:
            assert blocks.size == n_out * ((n_in + 255) // 256) * (144 if fmt == FMT_Q4K else 210)
        h = C.c_void_p()
        name = {FMT_Q4K: "pgd_matrix_upload_q4k", FMT_Q6K: "pgd_matrix_upload_q6k", FMT_Q8_0: "pgd_matrix_upload_q8_0",
                FMT_Q5_0: "pgd_matrix_upload_q5_0"}[fmt]
        call(name, dev.handle, _ptr(blocks), n_out, n_in, C.byref(h))
        return cls(dev, h)

    @classmethod
    def synth(cls, dev: Device, fmt: int, n_out: int, n_in: int, seed: int, key: int, std: float = 0.02):
        h = C.c_void_p()
        call("pgd_matrix_synth", dev.handle, fmt, n_out, n_in, C.c_uint64(seed), C.c_uint64(key), C.c_float(std), C.byref(h))
        return cls(dev, h)

    def free(self) -> None:
        if self.handle:
            call("pgd_matrix_free", self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    # ---- ops ----
    def dequant(self, row0: int = 0, rows: int | None = None) -> np.ndarray:
        rows = self.n_out - row0 if rows is None else rows
        out = np.empty((rows, self.n_in), np.float32)
        call("pgd_matrix_dequant", self.handle, row0, rows, _ptr(out))
        return out

    def gemv(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        squeeze = x.ndim == 1
        x2 = x.reshape(-1, self.n_in)
        y = np.empty((x2.shape[0], self.n_out), np.float32)
        call("pgd_matrix_gemv", self.handle, _ptr(x2), x2.shape[0], _ptr(y))
        return y[0] if squeeze else y

    def gemv_dev(self, x_ptr: int, ldx: int, nrows: int, y_ptr: int, ldy: int, x_f16: bool = False,
                 res_ptr: int = 0, ldres: int = 0) -> None:
        call("pgd_matrix_gemv_dev", self.handle, C.c_void_p(x_ptr), int(x_f16), ldx, nrows, C.c_void_p(y_ptr), ldy,
             C.c_void_p(res_ptr or None), ldres)

    def gemv_q8act_dev(self, x_ptr: int, ldx: int, nrows: int, y_ptr: int, ldy: int, res_ptr: int = 0,
                       ldres: int = 0) -> None:
        """candle's CPU quantized matmul arithmetic (activations quantized to Q8_K / Q8_0)."""
        call("pgd_matrix_gemv_q8act_dev", self.handle, C.c_void_p(x_ptr), ldx, nrows, C.c_void_p(y_ptr), ldy,
             C.c_void_p(res_ptr or None), ldres)

    def gemv_q8act_pair_dev(self, ya_ptr: int, other: "Matrix", yb_ptr: int, x_ptr: int, ldx: int, nrows: int,
                            ldy: int) -> None:
        """This matrix and `other` over the same rows in one launch (candle's CPU arithmetic)."""
        call("pgd_matrix_gemv_q8act_pair_dev", self.handle, C.c_void_p(ya_ptr), other.handle, C.c_void_p(yb_ptr),
             C.c_void_p(x_ptr), ldx, nrows, ldy)

    def gemv_act_dev(self, act_ptr: int, nrows: int, y_ptr: int, ldy: int, res_ptr: int = 0, ldres: int = 0) -> None:
        call("pgd_matrix_gemv_act_dev", self.handle, C.c_void_p(act_ptr), nrows, C.c_void_p(y_ptr), ldy,
             C.c_void_p(res_ptr or None), ldres)

    @staticmethod
    def gemv_swiglu_act_dev(gate: "Matrix", up: "Matrix", act_ptr: int, nrows: int, mid_ptr: int, ldm: int):
        call("pgd_matrix_gemv_swiglu_act_dev", gate.handle, up.handle, C.c_void_p(act_ptr), nrows, C.c_void_p(mid_ptr), ldm)

    @staticmethod
    def gemv_swiglu_dev(gate: "Matrix", up: "Matrix", x_ptr: int, ldx: int, nrows: int, mid_ptr: int, ldm: int):
        call("pgd_matrix_gemv_swiglu_dev", gate.handle, up.handle, C.c_void_p(x_ptr), ldx, nrows, C.c_void_p(mid_ptr), ldm)
