"""ctypes wrapper of oracle/_build/liboracle.so (TEST INFRASTRUCTURE ONLY).

The C restatement in oracle.c is the checker; this module only marshals
numpy arrays. Builds the library with `make -C oracle` when it is missing.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from dataclasses import dataclass, fields
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_lib = None

# tensor kinds of the synthetic generator: key = (layer << 8) | kind, layer
# 0xFFFF for model-global tensors
K_EMBED, K_HEAD, K_FINAL_NORM = 1, 2, 3
K_IN_NORM, K_POST_NORM, K_GATE, K_UP, K_DOWN = 10, 11, 12, 13, 14
K_QKV, K_Z, K_A, K_B, K_OUT, K_CONV, K_ALOG, K_DTB, K_GNORM = 20, 21, 22, 23, 24, 25, 26, 27, 28
K_Q, K_K, K_V, K_O, K_QNORM, K_KNORM, K_QB, K_KB, K_VB = 30, 31, 32, 33, 34, 35, 36, 37, 38


def tkey(layer: int, kind: int) -> int:
    return ((0xFFFF if layer < 0 else layer) << 8) | kind


def build() -> Path:
    r = subprocess.run(["make", "-s", "-C", str(HERE)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stderr)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _lib.ora_f32_to_bf16.restype = C.c_uint16
        _lib.ora_f32_to_bf16.argtypes = [C.c_float]
        _lib.ora_bf16_to_f32.restype = C.c_float
        _lib.ora_bf16_to_f32.argtypes = [C.c_uint16]
        _lib.ora_f32_to_f16.restype = C.c_uint16
        _lib.ora_f32_to_f16.argtypes = [C.c_float]
        _lib.ora_f16_to_f32.restype = C.c_float
        _lib.ora_f16_to_f32.argtypes = [C.c_uint16]
        _lib.ora_synth_normal.restype = C.c_float
        _lib.ora_synth_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        _lib.ora_synth_uniform.restype = C.c_float
        _lib.ora_synth_uniform.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        _lib.ora_synth_normal_fill.argtypes = [C.c_uint64, C.c_uint64, C.c_float, C.c_void_p, C.c_size_t]
        _lib.ora_kq_blocks.restype = C.c_int
        for n in ("ora_qwen35_new", "ora_qwen35_cache_new", "ora_qwen35_cache_clone", "ora_qwen2_new",
                  "ora_qwen2_cache_new", "ora_qwen35_tensor", "ora_qwen2_tensor"):
            getattr(_lib, n).restype = C.c_void_p
        _lib.ora_qwen35_new.argtypes = [C.c_void_p, C.c_uint64]
        _lib.ora_qwen2_new.argtypes = [C.c_void_p, C.c_uint64]
        for n in ("ora_qwen35_free", "ora_qwen35_cache_free", "ora_qwen2_free", "ora_qwen2_cache_free"):
            getattr(_lib, n).argtypes = [C.c_void_p]
        _lib.ora_qwen35_cache_new.argtypes = [C.c_void_p]
        _lib.ora_qwen35_cache_clone.argtypes = [C.c_void_p]
        _lib.ora_qwen2_cache_new.argtypes = [C.c_void_p]
        _lib.ora_qwen35_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
        _lib.ora_qwen35_forward_all.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
        _lib.ora_qwen2_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
        _lib.ora_qwen35_tensor.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int]
        _lib.ora_qwen2_tensor.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int]
        _lib.ora_qwen2_set_matrix.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]
        for n in ("ora_q8_0_dequant", "ora_q5_0_dequant"):
            getattr(_lib, n).argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]
        _lib.ora_qwen35_cache_to_bytes.restype = C.c_size_t
        _lib.ora_qwen35_cache_to_bytes.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        _lib.ora_qwen35_cache_from_bytes.restype = C.c_void_p
        _lib.ora_qwen35_cache_from_bytes.argtypes = [C.c_void_p, C.c_size_t]
        _lib.ora_qwen2_cache_len.restype = C.c_int
        _lib.ora_qwen2_cache_len.argtypes = [C.c_void_p]
        _lib.ora_qwen2_cache_export.restype = C.c_size_t
        _lib.ora_qwen2_cache_export.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                                C.c_size_t]
        _lib.ora_qwen2_cache_import.restype = C.c_void_p
        _lib.ora_qwen2_cache_import.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_int,
                                                C.c_void_p]
        _lib.ora_qwen35_cache_len.restype = C.c_int
        _lib.ora_qwen35_cache_len.argtypes = [C.c_void_p]
        _lib.ora_argmax_first.restype = C.c_uint32
        _lib.ora_argmax_first.argtypes = [C.c_void_p, C.c_int]
        _lib.ora_q8k_quantize.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
        _lib.ora_kq_vec_dot_q8k.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        _lib.ora_qwen2_set_kquant_mode.argtypes = [C.c_void_p, C.c_int]
        _lib.ora_q8_0_quantize_act.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
        _lib.ora_q8_0_vec_dot.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        _lib.ora_num_threads.restype = C.c_int
        _lib.ora_exp_rows.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
        _lib.ora_rope_cos_sin.argtypes = [C.c_int, C.c_int, C.c_float, C.c_void_p, C.c_void_p]
    return _lib


def _p(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------------------
# formats
# ---------------------------------------------------------------------------
def synth_normal(seed: int, key: int, n: int, scale: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().ora_synth_normal_fill(seed, key, scale, _p(out), n)
    return out


def synth_uniform(seed: int, key: int, idx: int) -> float:
    return lib().ora_synth_uniform(seed, key, idx)


def a8_quantize(w: np.ndarray):
    w = np.ascontiguousarray(w, np.float32)
    n_out, n_in = w.shape
    packed = np.zeros(n_out * n_in // 4, np.uint32)
    scales = np.zeros(n_out * (n_in // 64), np.uint16)
    biases = np.zeros_like(scales)
    lib().ora_a8_quantize(_p(w), n_out, n_in, _p(packed), _p(scales), _p(biases))
    return packed, scales, biases


def a8_dequant(packed, scales, biases, n_out: int, n_in: int) -> np.ndarray:
    out = np.empty((n_out, n_in), np.float32)
    lib().ora_a8_dequant(_p(np.ascontiguousarray(packed, np.uint32)), _p(np.ascontiguousarray(scales, np.uint16)),
                         _p(np.ascontiguousarray(biases, np.uint16)), 0, n_out, n_in, _p(out))
    return out


def kq_blocks(n_in: int) -> int:
    return (n_in + 255) // 256


def q4k_quantize(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    n_out, n_in = w.shape
    out = np.zeros(n_out * kq_blocks(n_in) * 144, np.uint8)
    lib().ora_q4k_quantize(_p(w), n_out, n_in, _p(out))
    return out


def q6k_quantize(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    n_out, n_in = w.shape
    out = np.zeros(n_out * kq_blocks(n_in) * 210, np.uint8)
    lib().ora_q6k_quantize(_p(w), n_out, n_in, _p(out))
    return out


def q4k_dequant(blocks: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    out = np.empty((n_out, n_in), np.float32)
    lib().ora_q4k_dequant(_p(np.ascontiguousarray(blocks, np.uint8)), 0, n_out, n_in, _p(out))
    return out


def q6k_dequant(blocks: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    out = np.empty((n_out, n_in), np.float32)
    lib().ora_q6k_dequant(_p(np.ascontiguousarray(blocks, np.uint8)), 0, n_out, n_in, _p(out))
    return out


def q8_0_dequant(blocks: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    out = np.empty((n_out, n_in), np.float32)
    lib().ora_q8_0_dequant(_p(np.ascontiguousarray(blocks, np.uint8)), 0, n_out, n_in, _p(out))
    return out


def q5_0_dequant(blocks: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    out = np.empty((n_out, n_in), np.float32)
    lib().ora_q5_0_dequant(_p(np.ascontiguousarray(blocks, np.uint8)), 0, n_out, n_in, _p(out))
    return out


def f32_to_bf16(x: float) -> int:
    return lib().ora_f32_to_bf16(x)


def bf16_to_f32(h: int) -> float:
    return lib().ora_bf16_to_f32(h)


Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])


def q8k_quantize(x: np.ndarray) -> np.ndarray:
    """candle's BlockQ8K::from_float of one activation row (tail padded with
    zeros) -> structured array of blocks (d, qs, bsums)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(kq_blocks(x.size) * 292, np.uint8)
    lib().ora_q8k_quantize(_p(x), x.size, _p(out))
    return out.view(Q8K_DTYPE)


def exp_f32(x: np.ndarray) -> np.ndarray:
    """e^x as the oracle's f32 paths evaluate it (double exponential rounded once)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().ora_exp_rows(_p(x), int(x.size), _p(y))
    return y


def kq_vec_dot_q8k(fmt: int, blocks: np.ndarray, n_out: int, n_in: int, q8k: np.ndarray) -> np.ndarray:
    """candle's CPU Q4_K (fmt 1) / Q6_K (fmt 2) x Q8_K block dot per weight row."""
    y = np.empty(n_out, np.float32)
    q = np.ascontiguousarray(q8k).view(np.uint8)
    lib().ora_kq_vec_dot_q8k(fmt, _p(np.ascontiguousarray(blocks, np.uint8)), n_out, n_in, _p(q), _p(y))
    return y


Q8_0_ACT_DTYPE = np.dtype([("d", "<u2"), ("qs", "i1", 32)])


def q8_0_quantize_act(x: np.ndarray) -> np.ndarray:
    """candle's BlockQ8_0::from_float of one activation row -> blocks (d f16 bits, qs)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(x.size // 32 * 34, np.uint8)
    lib().ora_q8_0_quantize_act(_p(x), x.size, _p(out))
    return out.view(Q8_0_ACT_DTYPE)


def q8_0_vec_dot(fmt: int, blocks: np.ndarray, n_out: int, n_in: int, q8: np.ndarray) -> np.ndarray:
    """candle's CPU Q8_0 (fmt 3) / Q5_0 (fmt 4) x Q8_0 block dot per weight row."""
    y = np.empty(n_out, np.float32)
    q = np.ascontiguousarray(q8).view(np.uint8)
    lib().ora_q8_0_vec_dot(fmt, _p(np.ascontiguousarray(blocks, np.uint8)), n_out, n_in, _p(q), _p(y))
    return y


def f32_to_f16(x: float) -> int:
    return lib().ora_f32_to_f16(x)


def f16_to_f32(h: int) -> float:
    return lib().ora_f16_to_f32(h)


# ---------------------------------------------------------------------------
# ops
# ---------------------------------------------------------------------------
def gdn_step(conv_out, a, b, z, a_log, dt_bias, norm, k_heads, v_heads, k_dim, v_dim, state):
    """Sequential recurrence over seq tokens; state updated in place."""
    conv_out = np.ascontiguousarray(conv_out, np.float32)
    seq = conv_out.shape[0]
    out = np.zeros((seq, v_heads * v_dim), np.float32)
    arrs = [np.ascontiguousarray(v, np.float32) for v in (a, b, z, a_log, dt_bias, norm)]
    assert state.dtype == np.float32 and state.flags.c_contiguous
    lib().ora_gdn_step(_p(conv_out), *map(_p, arrs), seq, k_heads, v_heads, k_dim, v_dim, _p(state), _p(out))
    return out


def attn_decode(q, k_cache, v_cache, length, heads, kv_heads, hd, gate=None):
    q = np.ascontiguousarray(q, np.float32)
    k_cache = np.ascontiguousarray(k_cache, np.float32)
    v_cache = np.ascontiguousarray(v_cache, np.float32)
    out = np.zeros((heads, hd), np.float32)
    g = None if gate is None else np.ascontiguousarray(gate, np.float32)
    lib().ora_attn_decode(_p(q), _p(k_cache), _p(v_cache), length, heads, kv_heads, hd,
                          _p(g) if g is not None else None, _p(out))
    return out


def causal_conv(x, kernel, weight, state):
    x = np.ascontiguousarray(x, np.float32)
    seq, channels = x.shape
    out = np.zeros_like(x)
    lib().ora_causal_conv(_p(x), seq, channels, kernel, _p(np.ascontiguousarray(weight, np.float32)), _p(state), _p(out))
    return out


def rope_cos_sin(pos: int, rotary_dim: int, theta: float):
    c = np.zeros(rotary_dim, np.float32)
    s = np.zeros(rotary_dim, np.float32)
    lib().ora_rope_cos_sin(pos, rotary_dim, C.c_float(theta), _p(c), _p(s))
    return c, s


def argmax_first(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().ora_argmax_first(_p(x), x.size))


# ---------------------------------------------------------------------------
# models
# ---------------------------------------------------------------------------
class _Q35Cfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "hidden", "intermediate", "vocab", "heads", "kv_heads",
                                       "head_dim", "rotary_dim")] + [("rope_theta", C.c_float)] + \
               [(n, C.c_int) for n in ("k_heads", "v_heads", "k_dim", "v_dim", "conv_kernel", "full_every")]


class _Q2Cfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "hidden", "intermediate", "vocab", "heads", "kv_heads",
                                       "head_dim", "max_pos")] + [("rope_theta", C.c_float), ("eps", C.c_float)]


@dataclass
class Qwen35Config:
    n_layers: int = 64
    hidden: int = 5120
    intermediate: int = 17408
    vocab: int = 151936
    heads: int = 24
    kv_heads: int = 4
    head_dim: int = 256
    rotary_dim: int = 64
    rope_theta: float = 1e7
    k_heads: int = 16
    v_heads: int = 32
    k_dim: int = 128
    v_dim: int = 128
    conv_kernel: int = 4
    full_every: int = 4

    def ctype(self):
        return _Q35Cfg(**{f.name: getattr(self, f.name) for f in fields(self)})


@dataclass
class Qwen2Config:
    n_layers: int = 24
    hidden: int = 896
    intermediate: int = 4864
    vocab: int = 151936
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    max_pos: int = 32768
    rope_theta: float = 1e6
    eps: float = 1e-6

    def ctype(self):
        return _Q2Cfg(**{f.name: getattr(self, f.name) for f in fields(self)})


class Qwen35:
    """CPU restatement of Qwen35 (pagoda-hf/src/qwen3_5.rs) on synthetic weights."""

    def __init__(self, cfg: Qwen35Config, seed: int):
        self.cfg = cfg
        self._c = cfg.ctype()
        self.h = lib().ora_qwen35_new(C.byref(self._c), seed)

    def new_cache(self):
        return Qwen35Cache(self, lib().ora_qwen35_cache_new(self.h))

    def forward(self, toks, cache) -> np.ndarray:
        t = np.ascontiguousarray(toks, np.uint32)
        out = np.empty(self.cfg.vocab, np.float32)
        rc = lib().ora_qwen35_forward(self.h, _p(t), t.size, cache.h, _p(out))
        if rc:
            raise ValueError(f"oracle forward failed {rc}")
        return out

    def forward_all(self, toks, cache) -> np.ndarray:
        t = np.ascontiguousarray(toks, np.uint32)
        out = np.empty((t.size, self.cfg.vocab), np.float32)
        rc = lib().ora_qwen35_forward_all(self.h, _p(t), t.size, cache.h, _p(out))
        if rc:
            raise ValueError(f"oracle forward failed {rc}")
        return out

    def tensor_ptr(self, layer: int, kind: int, part: int = 0) -> int:
        return lib().ora_qwen35_tensor(self.h, layer, kind, part)

    def __del__(self):
        try:
            lib().ora_qwen35_free(self.h)
        except Exception:
            pass


class Qwen35Cache:
    def __init__(self, model, h):
        self.model, self.h = model, h

    def clone(self):
        return Qwen35Cache(self.model, lib().ora_qwen35_cache_clone(self.h))

    def __len__(self):
        return lib().ora_qwen35_cache_len(self.h)

    @classmethod
    def from_bytes(cls, blob: bytes, model=None):
        """Cache v1 bytes -> oracle cache (qwen3_5.rs:208-256); ValueError if malformed."""
        buf = np.frombuffer(bytes(blob), np.uint8).copy()
        h = lib().ora_qwen35_cache_from_bytes(_p(buf) if buf.size else None, buf.size)
        if not h:
            raise ValueError("malformed cache v1 bytes")
        return cls(model, h)

    def to_bytes(self) -> bytes:
        n = lib().ora_qwen35_cache_to_bytes(self.h, None, 0)
        buf = np.zeros(n, np.uint8)
        lib().ora_qwen35_cache_to_bytes(self.h, _p(buf), n)
        return buf.tobytes()

    def __del__(self):
        try:
            lib().ora_qwen35_cache_free(self.h)
        except Exception:
            pass


class Qwen2:
    """CPU restatement of Qwen2Gguf (pagoda-hf/src/qwen2_gguf.rs) on synthetic weights."""

    def __init__(self, cfg: Qwen2Config, seed: int, kquant_mode: int = 1):
        """kquant_mode 1 (default): the reference CPU path's arithmetic,
        candle's quantized matmul (activations quantized to Q8_K / Q8_0);
        0: f32 dequant-then-dot."""
        self.cfg = cfg
        self._c = cfg.ctype()
        self.h = lib().ora_qwen2_new(C.byref(self._c), seed)
        self.set_kquant_mode(kquant_mode)

    def set_kquant_mode(self, mode: int) -> None:
        self.kquant_mode = int(mode)
        lib().ora_qwen2_set_kquant_mode(self.h, self.kquant_mode)

    def new_cache(self):
        return Qwen2Cache(lib().ora_qwen2_cache_new(self.h), self)

    def forward(self, toks, cache) -> np.ndarray:
        t = np.ascontiguousarray(toks, np.uint32)
        out = np.empty(self.cfg.vocab, np.float32)
        rc = lib().ora_qwen2_forward(self.h, _p(t), t.size, cache.h, _p(out))
        if rc:
            raise ValueError(f"oracle forward failed {rc}")
        return out

    def tensor_ptr(self, layer: int, kind: int, part: int = 0) -> int:
        return lib().ora_qwen2_tensor(self.h, layer, kind, part)

    def set_matrix(self, layer: int, kind: int, fmt: int, blocks: np.ndarray) -> None:
        """Replace one matrix by GGML blocks (fmt 1 Q4_K, 2 Q6_K, 3 Q8_0, 4 Q5_0)."""
        b = np.ascontiguousarray(blocks, np.uint8)
        if lib().ora_qwen2_set_matrix(self.h, layer, kind, fmt, _p(b)):
            raise ValueError("ora_qwen2_set_matrix rejected the matrix")

    def __del__(self):
        try:
            lib().ora_qwen2_free(self.h)
        except Exception:
            pass


class Qwen2Cache:
    def __init__(self, h, model=None):
        self.h, self.model = h, model

    def __len__(self):
        return lib().ora_qwen2_cache_len(self.h)

    def export_bytes(self, logits=None, f16: bool = False) -> bytes:
        """SessionKv::export_bytes (pagoda-hf/src/llama.rs:215-266)."""
        lg = None if logits is None else np.ascontiguousarray(logits, np.float32)
        args = (self.model.h, self.h, _p(lg) if lg is not None else None, 0 if lg is None else lg.size, int(f16))
        n = lib().ora_qwen2_cache_export(*args, None, 0)
        buf = np.zeros(n, np.uint8)
        lib().ora_qwen2_cache_export(*args, _p(buf), n)
        return buf.tobytes()

    @classmethod
    def import_bytes(cls, model, blob: bytes):
        """SessionKv::import_bytes (llama.rs:268-345) -> (cache, logits or None)."""
        buf = np.frombuffer(bytes(blob), np.uint8).copy()
        lg = np.zeros(model.cfg.vocab, np.float32)
        nl = C.c_int(0)
        h = lib().ora_qwen2_cache_import(model.h, _p(buf) if buf.size else None, buf.size, _p(lg), lg.size,
                                         C.byref(nl))
        if not h:
            raise ValueError("malformed SessionKv payload")
        return cls(h, model), (lg[:nl.value].copy() if nl.value else None)

    def __del__(self):
        try:
            lib().ora_qwen2_cache_free(self.h)
        except Exception:
            pass
_Q2Cache = Qwen2Cache
