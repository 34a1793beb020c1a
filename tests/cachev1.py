"""Reader of the hybrid model's cache bytes v1 (pagoda-hf/src/qwen3_5.rs:177-256),
written from the format's definition for the tests: u32 version (1), u64
len, u32 n_layers; per layer a tag byte, 1 = linear (counted f32 vectors
conv, state), 2 = full (u32 kv_len, kv_heads, head_dim, counted f32 k, v).
A counted vector is a u32 count then count little-endian f32."""
from __future__ import annotations

import struct

import numpy as np


def parse(blob: bytes) -> dict:
    at = 0

    def take(fmt):
        nonlocal at
        n = struct.calcsize(fmt)
        if at + n > len(blob):
            raise ValueError("truncated")
        v = struct.unpack_from(fmt, blob, at)
        at += n
        return v[0] if len(v) == 1 else v

    def vec():
        nonlocal at
        n = take("<I")
        if at + 4 * n > len(blob):
            raise ValueError("truncated vector")
        a = np.frombuffer(blob, "<f4", n, at).copy()
        at += 4 * n
        return a

    version = take("<I")
    if version != 1:
        raise ValueError(f"version {version}")
    out = {"len": take("<Q"), "layers": []}
    for _ in range(take("<I")):
        tag = take("<B")
        if tag == 1:
            out["layers"].append({"tag": 1, "conv": vec(), "state": vec()})
        elif tag == 2:
            kv_len, kvh, hd = take("<III")
            k, v = vec(), vec()
            if k.size != kv_len * kvh * hd or v.size != k.size:
                raise ValueError("kv shape")
            out["layers"].append({"tag": 2, "kv_len": kv_len, "kv_heads": kvh, "head_dim": hd, "k": k, "v": v})
        else:
            raise ValueError(f"tag {tag}")
    if at != len(blob):
        raise ValueError("trailing bytes")
    return out
