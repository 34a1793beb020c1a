"""ctypes binding of libpagoda_hip.so (the C ABI in include/pagoda_hip.h).

The library is the product: there is no CPU fallback. If the shared object
is missing or cannot be loaded this module raises, on every machine.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libpagoda_hip.so"

c_int, c_float, c_double, c_size_t, c_void_p, c_char_p = C.c_int, C.c_float, C.c_double, C.c_size_t, C.c_void_p, C.c_char_p
c_uint64, c_uint32 = C.c_uint64, C.c_uint32
P = C.POINTER

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple] = {
    "pgd_last_error": (c_int, [c_char_p, c_size_t]),
    "pgd_version": (c_int, []),
    "pgd_device_open": (c_int, [c_char_p, P(c_void_p)]),
    "pgd_device_close": (c_int, [c_void_p]),
    "pgd_device_sync": (c_int, [c_void_p]),
    "pgd_device_stream": (c_void_p, [c_void_p]),
    "pgd_device_malloc": (c_int, [c_void_p, c_size_t, P(c_void_p)]),
    "pgd_device_free": (c_int, [c_void_p, c_void_p]),
    "pgd_device_memcpy": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_int]),
    "pgd_device_copy_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
    "pgd_event_new": (c_int, [c_void_p, P(c_void_p)]),
    "pgd_event_record": (c_int, [c_void_p]),
    "pgd_event_elapsed_ms": (c_int, [c_void_p, c_void_p, P(c_float)]),
    "pgd_event_free": (c_int, [c_void_p]),
    "pgd_matrix_upload_a8": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, P(c_void_p)]),
    "pgd_matrix_upload_q4k": (c_int, [c_void_p, c_void_p, c_int, c_int, P(c_void_p)]),
    "pgd_matrix_upload_q6k": (c_int, [c_void_p, c_void_p, c_int, c_int, P(c_void_p)]),
    "pgd_matrix_upload_q8_0": (c_int, [c_void_p, c_void_p, c_int, c_int, P(c_void_p)]),
    "pgd_matrix_upload_q5_0": (c_int, [c_void_p, c_void_p, c_int, c_int, P(c_void_p)]),
    "pgd_matrix_synth": (c_int, [c_void_p, c_int, c_int, c_int, c_uint64, c_uint64, c_float, P(c_void_p)]),
    "pgd_matrix_free": (c_int, [c_void_p]),
    "pgd_matrix_info": (c_int, [c_void_p, P(c_int), P(c_int), P(c_int), P(c_size_t), P(c_double)]),
    "pgd_matrix_dequant": (c_int, [c_void_p, c_int, c_int, c_void_p]),
    "pgd_matrix_gemv": (c_int, [c_void_p, c_void_p, c_int, c_void_p]),
    "pgd_matrix_gemv_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_int, c_void_p, c_int]),
    "pgd_matrix_gemv_swiglu_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_int]),
    "pgd_gdn_step_dev": (c_int, [c_void_p, c_int, c_int] + [c_void_p] * 10 + [c_int, c_void_p]),
    "pgd_gdn_prefill_dev": (c_int, [c_void_p, c_int, c_int] + [c_void_p] * 10 + [c_int, c_int, c_int, c_void_p]),
    "pgd_attn_decode_dev": (c_int, [c_void_p, c_int, c_int, c_int, c_int] + [c_void_p] * 7 + [c_int, c_int, c_void_p]),
    "pgd_act_bytes": (c_size_t, [c_int, c_int]),
    "pgd_act_prep_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "pgd_matrix_gemv_act_dev": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p, c_int]),
    "pgd_matrix_gemv_q8act_dev": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_int]),
    "pgd_matrix_gemv_q8act_pair_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int]),
    "pgd_model_set_kquant_arith": (c_int, [c_void_p, c_int]),
    "pgd_matrix_gemv_act_dev_noalloc": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p, c_int]),
    "pgd_noalloc_scratch_bytes": (c_size_t, []),
    "pgd_matrix_gemv_swiglu_act_dev": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int]),
    "pgd_model_synth": (c_int, [c_void_p, c_void_p, c_uint64, P(c_void_p)]),
    "pgd_model_load_mlx": (c_int, [c_void_p, c_char_p, c_int, c_int, P(c_void_p)]),
    "pgd_model_load_gguf": (c_int, [c_void_p, c_char_p, c_int, c_int, P(c_void_p)]),
    "pgd_checkpoint_config": (c_int, [c_char_p, c_int, c_int, c_void_p]),
    "pgd_model_config_get": (c_int, [c_void_p, c_void_p]),
    "pgd_model_free": (c_int, [c_void_p]),
    "pgd_model_set_graphs": (c_int, [c_void_p, c_int]),
    "pgd_model_graph_stats": (c_int, [c_void_p, P(c_int), P(C.c_longlong)]),
    "pgd_model_info": (c_int, [c_void_p, P(c_size_t), P(c_double), P(c_int)]),
    "pgd_session_new": (c_int, [c_void_p, P(c_void_p)]),
    "pgd_session_fork": (c_int, [c_void_p, P(c_void_p)]),
    "pgd_session_fork_prefix": (c_int, [c_void_p, c_int, P(c_void_p)]),
    "pgd_set_kv_wire_f16": (c_int, [c_int]),
    "pgd_model_kv_pool": (c_int, [c_void_p, P(c_int), P(c_int), P(c_int)]),
    "pgd_session_pages": (c_int, [c_void_p, c_void_p, c_int, P(c_int)]),
    "pgd_page_retain": (c_int, [c_void_p, c_void_p, c_int]),
    "pgd_page_release": (c_int, [c_void_p, c_void_p, c_int]),
    "pgd_page_refcount": (c_int, [c_void_p, C.c_int32, P(c_int)]),
    "pgd_session_from_pages": (c_int, [c_void_p, c_void_p, c_int, c_int, P(c_void_p)]),
    "pgd_session_free": (c_int, [c_void_p]),
    "pgd_session_len": (c_int, [c_void_p, P(c_int)]),
    "pgd_forward": (c_int, [c_void_p, c_void_p, c_int, c_void_p]),
    "pgd_forward_greedy": (c_int, [c_void_p, c_uint32, P(c_uint32), P(c_float)]),
    "pgd_forward_verify": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "pgd_step_ragged": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "pgd_session_export": (c_int, [c_void_p, c_void_p, c_size_t, P(c_size_t)]),
    "pgd_session_import": (c_int, [c_void_p, c_void_p, c_size_t, P(c_void_p)]),
}

_lib: C.CDLL | None = None


class PagodaError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"pagoda_hip error {code}: {msg}")
        self.code = code


def lib() -> C.CDLL:
    """Load the backend library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(the HIP backend has no CPU fallback)")
        l = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def last_error() -> str:
    buf = C.create_string_buffer(4096)
    lib().pgd_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc: int) -> None:
    if rc != 0:
        raise PagodaError(rc, last_error())


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
