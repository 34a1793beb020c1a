"""Reader and writer of the SessionKv PD payload (pagoda-hf/src/llama.rs:
215-345), written from the format's definition for the tests: u32 magic
0x50444B56, version (1: payload f32; 2: the dtype field selects f32 (0) or
f16 (1)), token count, layer count, logits (u32 count + f32), then per layer
u32 present; when present u32 kv_heads, head_dim, dtype and K then V as
[kv_heads, len, head_dim]."""
from __future__ import annotations

import struct

import numpy as np

MAGIC = 0x50444B56


def parse(blob: bytes) -> dict:
    at = 0

    def u32():
        nonlocal at
        if at + 4 > len(blob):
            raise ValueError("truncated")
        v = struct.unpack_from("<I", blob, at)[0]
        at += 4
        return v

    def arr(dt, n):
        nonlocal at
        size = np.dtype(dt).itemsize * n
        if at + size > len(blob):
            raise ValueError("truncated")
        a = np.frombuffer(blob, dt, n, at).copy()
        at += size
        return a

    if u32() != MAGIC:
        raise ValueError("magic")
    version = u32()
    if version not in (1, 2):
        raise ValueError(f"version {version}")
    out = {"version": version, "len": u32(), "layers": []}
    n_layers = u32()
    out["logits"] = arr("<f4", u32())
    for _ in range(n_layers):
        if u32() == 0:
            out["layers"].append(None)
            continue
        kvh, hd, dt = u32(), u32(), u32()
        f16 = version >= 2 and dt == 1
        n = kvh * out["len"] * hd
        kv = [arr("<f2" if f16 else "<f4", n).reshape(kvh, out["len"], hd) for _ in range(2)]
        out["layers"].append({"kv_heads": kvh, "head_dim": hd, "dtype": dt, "k": kv[0], "v": kv[1]})
    out["trailing"] = len(blob) - at
    return out


def write(length: int, layers, logits=None, f16: bool = False, version: int = 2) -> bytes:
    """layers: list of None or (k, v) arrays shaped [kv_heads, length, head_dim]."""
    b = bytearray(struct.pack("<4I", MAGIC, version, length, len(layers)))
    lg = np.asarray([] if logits is None else logits, "<f4")
    b += struct.pack("<I", lg.size) + lg.tobytes()
    for L in layers:
        if L is None:
            b += struct.pack("<I", 0)
            continue
        k, v = (np.asarray(t, np.float32) for t in L)
        b += struct.pack("<4I", 1, k.shape[0], k.shape[2], 1 if f16 else 0)
        for t in (k, v):
            b += t.astype("<f2" if f16 else "<f4").tobytes()
    return bytes(b)
