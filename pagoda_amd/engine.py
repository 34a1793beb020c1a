"""Model / session surface over the C ABI, mirroring the reference's plugin
traits: ModelEngine and ModelSession (pagoda/src/model.rs:66-195), the
CandleCausalLM backend contract (pagoda-hf/src/lib.rs:199-249) and the
hybrid model's Qwen35 entry points (pagoda-hf/src/qwen3_5.rs:466-755).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, fields, replace

import numpy as np

from ._lib import PagodaError, call, last_error, lib
from .device import Device

ARCH_QWEN35, ARCH_QWEN2 = 0, 1
ARITH_DEQUANT_F32, ARITH_CPU_Q8 = 0, 1


class _Cfg(C.Structure):
    _fields_ = [("arch", C.c_int)] + [(n, C.c_int) for n in (
        "n_layers", "hidden", "intermediate", "vocab", "heads", "kv_heads", "head_dim", "rotary_dim")] + \
        [("rope_theta", C.c_float), ("eps", C.c_float)] + [(n, C.c_int) for n in (
            "k_heads", "v_heads", "k_dim", "v_dim", "conv_kernel", "full_every", "max_pos", "kv_block", "kv_blocks")]


@dataclass
class ModelConfig:
    arch: int = ARCH_QWEN35
    n_layers: int = 64
    hidden: int = 5120
    intermediate: int = 17408
    vocab: int = 151936
    heads: int = 24
    kv_heads: int = 4
    head_dim: int = 256
    rotary_dim: int = 64
    rope_theta: float = 1e7
    eps: float = 1e-6
    k_heads: int = 16
    v_heads: int = 32
    k_dim: int = 128
    v_dim: int = 128
    conv_kernel: int = 4
    full_every: int = 4
    max_pos: int = 32768
    kv_block: int = 16
    kv_blocks: int = 4096

    def ctype(self) -> _Cfg:
        return _Cfg(**{f.name: getattr(self, f.name) for f in fields(self)})


# Config 4: 27B-class hybrid (64 layers, 3:1 Gated-DeltaNet : full attention)
QWEN35_27B = ModelConfig()
# Config 1: Qwen2.5-0.5B architecture, GGUF Q4_K_M-style
QWEN2_05B = ModelConfig(arch=ARCH_QWEN2, n_layers=24, hidden=896, intermediate=4864, vocab=151936, heads=14,
                        kv_heads=2, head_dim=64, rotary_dim=64, rope_theta=1e6, eps=1e-6, k_heads=0, v_heads=0,
                        k_dim=0, v_dim=0, conv_kernel=0, full_every=1, max_pos=32768, kv_blocks=2048)


def _from_ctype(c: _Cfg) -> ModelConfig:
    return ModelConfig(**{f.name: getattr(c, f.name) for f in fields(ModelConfig)})


def _config_of(h: C.c_void_p) -> ModelConfig:
    c = _Cfg()
    call("pgd_model_config_get", h, C.byref(c))
    return _from_ctype(c)


def checkpoint_config(path: str, max_pos: int = 0, kv_blocks: int = 2048) -> ModelConfig:
    """The configuration pgd_model_load_mlx (a directory) or
    pgd_model_load_gguf (a file) derives from a checkpoint; needs no device."""
    c = _Cfg()
    call("pgd_checkpoint_config", str(path).encode(), int(max_pos), int(kv_blocks), C.byref(c))
    return _from_ctype(c)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32).reshape(-1))


def _p(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


class Model:
    """A model resident on one device (Qwen35 / Qwen2Gguf counterpart)."""

    def __init__(self, dev: Device, handle: C.c_void_p, cfg: ModelConfig):
        self.dev, self.handle, self.cfg = dev, handle, cfg

    @classmethod
    def synth(cls, dev: Device, cfg: ModelConfig, seed: int) -> "Model":
        h = C.c_void_p()
        c = cfg.ctype()
        call("pgd_model_synth", dev.handle, C.byref(c), C.c_uint64(seed), C.byref(h))
        return cls(dev, h, replace(cfg))

    @classmethod
    def load_mlx(cls, dev: Device, path: str, max_pos: int = 0, kv_blocks: int = 2048) -> "Model":
        """Qwen35::load (pagoda-hf/src/qwen3_5.rs:338-452): an MLX 8-bit model
        directory. max_pos 0: the config's max_position_embeddings."""
        h = C.c_void_p()
        call("pgd_model_load_mlx", dev.handle, str(path).encode(), int(max_pos), int(kv_blocks), C.byref(h))
        return cls(dev, h, _config_of(h))

    @classmethod
    def load_gguf(cls, dev: Device, path: str, max_pos: int = 0, kv_blocks: int = 2048) -> "Model":
        """Qwen2 GGUF load (pagoda-hf/src/qwen2_gguf.rs:65-140). max_pos 0:
        qwen2.context_length."""
        h = C.c_void_p()
        call("pgd_model_load_gguf", dev.handle, str(path).encode(), int(max_pos), int(kv_blocks), C.byref(h))
        return cls(dev, h, _config_of(h))

    def set_kquant_arith(self, mode: int) -> None:
        """ARITH_CPU_Q8 (the Qwen2 default: candle's CPU quantized matmul) or
        ARITH_DEQUANT_F32 for the GGML-format matrices."""
        call("pgd_model_set_kquant_arith", self.handle, int(mode))

    def set_graphs(self, on: bool) -> None:
        """Capture each step's launches into a HIP graph per launch signature
        and replay it on later steps of that signature (bitwise the same
        results as eager launches)."""
        call("pgd_model_set_graphs", self.handle, int(bool(on)))

    def graph_stats(self) -> dict:
        g, n = C.c_int(), C.c_longlong()
        call("pgd_model_graph_stats", self.handle, C.byref(g), C.byref(n))
        return {"graphs": g.value, "replays": n.value}

    def info(self) -> dict:
        wb, ab, kf = C.c_size_t(), C.c_double(), C.c_int()
        call("pgd_model_info", self.handle, C.byref(wb), C.byref(ab), C.byref(kf))
        return {"weight_bytes": wb.value, "algo_bytes_per_token": ab.value, "kv_free": kf.value}

    def free(self) -> None:
        if self.handle:
            call("pgd_model_free", self.handle)
            self.handle = C.c_void_p()

    @property
    def vocab_size(self) -> int:
        return self.cfg.vocab

    # ModelEngine::begin_session
    def new_session(self) -> "Session":
        h = C.c_void_p()
        call("pgd_session_new", self.handle, C.byref(h))
        return Session(self, h)

    def import_session(self, blob: bytes) -> "Session":
        buf = np.frombuffer(blob, np.uint8)
        h = C.c_void_p()
        call("pgd_session_import", self.handle, _p(buf), C.c_size_t(buf.size), C.byref(h))
        return Session(self, h)

    # ---- engine-addressable KV pages (pagoda/src/kv_cache.rs, radix_cache.rs) ----
    def kv_pool(self) -> dict:
        """PagedKvCache::num_blocks / block_size / num_free_blocks
        (pagoda/src/kv_cache.rs:48-56) of the device page pool."""
        n, b, f = C.c_int(), C.c_int(), C.c_int()
        call("pgd_model_kv_pool", self.handle, C.byref(n), C.byref(b), C.byref(f))
        return {"pages": n.value, "page_tokens": b.value, "free": f.value}

    def page_retain(self, ids) -> None:
        """PagedKvCache::inc_ref (kv_cache.rs:90) for each page id."""
        a = np.ascontiguousarray(ids, np.int32)
        call("pgd_page_retain", self.handle, _p(a) if a.size else None, int(a.size))

    def page_release(self, ids) -> None:
        """PagedKvCache::dec_ref (kv_cache.rs:95) for each page id."""
        a = np.ascontiguousarray(ids, np.int32)
        call("pgd_page_release", self.handle, _p(a) if a.size else None, int(a.size))

    def page_refcount(self, page: int) -> int:
        """PagedKvCache::ref_count (kv_cache.rs:74)."""
        n = C.c_int()
        call("pgd_page_refcount", self.handle, C.c_int32(int(page)), C.byref(n))
        return n.value

    def session_from_pages(self, ids, n_pos: int) -> "Session":
        """A session whose first n_pos positions are the KV held in `ids`
        (ceil(n_pos / page_tokens) pages, in position order): the radix
        cache's matched (BlockId, offset) slots (radix_cache.rs:17-18) made
        into a live cache without copying. Qwen2 only."""
        a = np.ascontiguousarray(ids, np.int32)
        h = C.c_void_p()
        call("pgd_session_from_pages", self.handle, _p(a) if a.size else None, int(a.size), int(n_pos),
             C.byref(h))
        return Session(self, h)

    def step_ragged(self, sessions, feeds, all_rows: bool = False, want_logits: bool = False):
        """One batched forward: session i feeds feeds[i] (>= 1 tokens).
        Returns (ids, logits|None); ids per session (last position) or per fed
        token when all_rows."""
        toks = _u32(np.concatenate([_u32(f) for f in feeds]))
        n = np.ascontiguousarray([len(f) for f in feeds], np.int32)
        rows = int(toks.size) if all_rows else len(feeds)
        ids = np.zeros(rows, np.uint32)
        logits = np.empty((rows, self.cfg.vocab), np.float32) if want_logits else None
        arr = (C.c_void_p * len(sessions))(*[s.handle.value for s in sessions])
        call("pgd_step_ragged", self.handle, arr, _p(toks), _p(n), len(sessions), int(all_rows), _p(ids),
             _p(logits) if logits is not None else None)
        return ids, logits


class Session:
    """ModelSession (pagoda/src/model.rs:163-195) over a device-resident cache."""

    def __init__(self, model: Model, handle: C.c_void_p):
        self.model, self.handle = model, handle

    def free(self) -> None:
        if self.handle:
            call("pgd_session_free", self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def context_len(self) -> int:
        n = C.c_int()
        call("pgd_session_len", self.handle, C.byref(n))
        return n.value

    def forward(self, new_tokens) -> np.ndarray:
        t = _u32(new_tokens)
        out = np.empty(self.model.cfg.vocab, np.float32)
        call("pgd_forward", self.handle, _p(t) if t.size else None, int(t.size), _p(out))
        return out

    def forward_greedy(self, tok: int) -> tuple[int, float]:
        i, v = C.c_uint32(), C.c_float()
        call("pgd_forward_greedy", self.handle, C.c_uint32(tok), C.byref(i), C.byref(v))
        return int(i.value), float(v.value)

    def forward_verify(self, toks) -> list[tuple[int, float]]:
        t = _u32(toks)
        ids = np.zeros(t.size, np.uint32)
        vals = np.zeros(t.size, np.float32)
        call("pgd_forward_verify", self.handle, _p(t), int(t.size), _p(ids), _p(vals))
        return [(int(a), float(b)) for a, b in zip(ids, vals)]

    def fork(self) -> "Session":
        h = C.c_void_p()
        call("pgd_session_fork", self.handle, C.byref(h))
        return Session(self.model, h)

    def fork_prefix(self, n: int) -> "Session":
        """CandleCausalLM::cache_prefix (pagoda-hf/src/lib.rs:219-226): the
        first n positions as a new session (Qwen2 only)."""
        h = C.c_void_p()
        call("pgd_session_fork_prefix", self.handle, int(n), C.byref(h))
        return Session(self.model, h)

    def pages(self) -> np.ndarray:
        """Page ids holding positions [0, context_len) in order; position p
        lives in slot p % page_tokens of pages[p // page_tokens]."""
        n = C.c_int()
        call("pgd_session_pages", self.handle, None, 0, C.byref(n))
        ids = np.zeros(n.value, np.int32)
        call("pgd_session_pages", self.handle, _p(ids) if ids.size else None, int(ids.size), C.byref(n))
        return ids

    def export_kv(self) -> bytes:
        n = C.c_size_t()
        call("pgd_session_export", self.handle, None, C.c_size_t(0), C.byref(n))
        buf = np.zeros(n.value, np.uint8)
        call("pgd_session_export", self.handle, _p(buf), C.c_size_t(buf.size), C.byref(n))
        return buf.tobytes()


def set_kv_wire_f16(on: bool) -> None:
    """set_kv_wire_f16 (pagoda-hf/src/llama.rs:133-136): the SessionKv
    export's K/V encoding, process-wide."""
    call("pgd_set_kv_wire_f16", int(bool(on)))


def argmax_first(logits: np.ndarray) -> int:
    """Engine sampler's greedy rule: first max over finite values
    (pagoda/src/sampler.rs:59-69)."""
    x = np.where(np.isfinite(logits), logits, -np.inf)
    return int(np.argmax(x))


class HipEngine:
    """ModelEngine (pagoda/src/model.rs:66-147) for PAGODA_DEVICE=hip.

    Errors from the backend surface as uniform (zero) logits plus a logged
    message, as CandleModel does (pagoda-hf/src/lib.rs:564-572); the engine
    faults requests whose logits are not finite (engine.rs:1278-1295)."""

    def __init__(self, model: Model):
        self.model = model
        self.errors: list[str] = []

    def vocab_size(self) -> int:
        return self.model.cfg.vocab

    def name(self) -> str:
        return "pagoda-hip-qwen35" if self.model.cfg.arch == ARCH_QWEN35 else "pagoda-hip-qwen2-gguf"

    def begin_session(self) -> Session:
        return self.model.new_session()

    def forward(self, tokens) -> np.ndarray:
        s = self.model.new_session()
        try:
            return s.forward(tokens)
        except PagodaError as e:
            self.errors.append(str(e))
            return np.zeros(self.model.cfg.vocab, np.float32)
        finally:
            s.free()

    def session_forward_batch(self, sessions, feeds):
        """Batched decode: every feed is one or more fresh tokens. Atomic:
        on failure no session advances and None is returned (the engine then
        falls back to per-session forwards, engine.rs:493-501)."""
        if len(sessions) < 1:
            return None
        try:
            _, logits = self.model.step_ragged(sessions, feeds, all_rows=False, want_logits=True)
        except PagodaError as e:
            self.errors.append(str(e))
            return None
        return [logits[i] for i in range(len(sessions))]

    def graft_session(self, session: Session, covered: int):
        """ModelEngine::graft_session (pagoda-hf/src/lib.rs:603-616) once the
        prefix store has found `session` covering `covered` prompt tokens:
        the session sliced to exactly that prefix, or None when the backend
        cannot slice (the hybrid model's recurrent state)."""
        try:
            return session.fork_prefix(covered)
        except PagodaError as e:
            self.errors.append(str(e))
            return None

    def import_session(self, tokens, kv: bytes):
        try:
            s = self.model.import_session(kv)
        except PagodaError as e:
            self.errors.append(str(e))
            return None
        if s.context_len() != len(tokens):
            s.free()
            return None
        return s
