"""Checkpoint writers for the loader tests: MLX model directories (safetensors
shards written by the safetensors package, config.json) and GGUF v3 files
(written here from the published GGUF layout: magic, version, counts,
metadata key/values, tensor infos, 32-byte aligned data). Weights come from
the CPU oracle's seeded models, which hold the same bytes the device
generator makes for Model.synth."""
from __future__ import annotations

import ctypes as C
import json
import struct
from pathlib import Path

import numpy as np

from oracle import pyoracle as ora

# tensor kinds (the (layer << 8) | kind keys of the synthetic generator)
K_EMBED, K_HEAD, K_FINAL_NORM = 1, 2, 3
K_IN_NORM, K_POST_NORM, K_GATE, K_UP, K_DOWN = 10, 11, 12, 13, 14
K_QKV, K_Z, K_A, K_B, K_OUT, K_CONV, K_ALOG, K_DTB, K_GNORM = 20, 21, 22, 23, 24, 25, 26, 27, 28
K_Q, K_K, K_V, K_O, K_QNORM, K_KNORM, K_QB, K_KB, K_VB = 30, 31, 32, 33, 34, 35, 36, 37, 38


def host_array(ptr: int, ctype, n: int) -> np.ndarray:
    """Writable numpy view of n elements at an oracle pointer."""
    return np.ctypeslib.as_array((ctype * n).from_address(ptr))


# ---------------------------------------------------------------------------
# MLX
# ---------------------------------------------------------------------------
def mlx_text_config(cfg, max_pos=None, layer_types=None) -> dict:
    kinds = layer_types or ["full_attention" if i % cfg.full_every == cfg.full_every - 1 else "linear_attention"
                            for i in range(cfg.n_layers)]
    t = {"hidden_size": cfg.hidden, "num_hidden_layers": cfg.n_layers, "intermediate_size": cfg.intermediate,
         "vocab_size": cfg.vocab, "num_attention_heads": cfg.heads, "num_key_value_heads": cfg.kv_heads,
         "head_dim": cfg.head_dim, "linear_num_key_heads": cfg.k_heads, "linear_num_value_heads": cfg.v_heads,
         "linear_key_head_dim": cfg.k_dim, "linear_value_head_dim": cfg.v_dim,
         "linear_conv_kernel_dim": cfg.conv_kernel, "rms_norm_eps": cfg.eps, "eos_token_id": 0,
         "rope_parameters": {"rope_theta": cfg.rope_theta, "partial_rotary_factor": cfg.rotary_dim / cfg.head_dim},
         "layer_types": kinds}
    if max_pos:
        t["max_position_embeddings"] = max_pos
    return t


def write_mlx_config(d: Path, text: dict, quant=None) -> None:
    q = quant if quant is not None else {"bits": 8, "group_size": 64, "mode": "affine"}
    d.mkdir(parents=True, exist_ok=True)
    (d / "config.json").write_text(json.dumps({"model_type": "qwen3_5", "text_config": text,
                                               "quantization_config": q}))


def write_safetensors_shards(d: Path, tensors: dict, nshards: int = 2) -> None:
    """tensors: name -> (dtype, numpy array); dtype "U32", "BF16" (uint16 bits), "F16" or "F32"."""
    import torch
    from safetensors.torch import save_file

    def tt(dtype, a):
        a = np.ascontiguousarray(a)
        if dtype == "BF16":
            return torch.from_numpy(a.astype(np.uint16)).view(torch.bfloat16)
        if dtype == "F16":
            return torch.from_numpy(a.astype(np.float16))
        if dtype == "U32":
            return torch.from_numpy(a.astype(np.uint32))
        return torch.from_numpy(a.astype(np.float32))

    names = sorted(tensors)
    weight_map = {}
    for s in range(nshards):
        fname = f"model-{s + 1:05d}-of-{nshards:05d}.safetensors"
        part = {n: tt(*tensors[n]) for n in names[s::nshards]}
        save_file(part, str(d / fname))
        weight_map.update({n: fname for n in part})
    (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))


def mlx_tensors_from_oracle(cfg, oracle) -> dict:
    """Every language_model.* tensor of the hybrid model, from the oracle."""
    H = cfg.hidden
    key_dim, value_dim = cfg.k_heads * cfg.k_dim, cfg.v_heads * cfg.v_dim
    conv_dim = 2 * key_dim + value_dim
    out = {}

    def affine(name, layer, kind, n_out, n_in):
        g = n_out * n_in // 64
        out[name + ".weight"] = ("U32", host_array(oracle.tensor_ptr(layer, kind, 0), C.c_uint32,
                                                   n_out * n_in // 4).reshape(n_out, n_in // 4).copy())
        out[name + ".scales"] = ("BF16", host_array(oracle.tensor_ptr(layer, kind, 1), C.c_uint16, g)
                                 .reshape(n_out, n_in // 64).copy())
        out[name + ".biases"] = ("BF16", host_array(oracle.tensor_ptr(layer, kind, 2), C.c_uint16, g)
                                 .reshape(n_out, n_in // 64).copy())

    def vec(name, layer, kind, n, dtype="F32", shape=None):
        a = host_array(oracle.tensor_ptr(layer, kind), C.c_float, n).copy()
        if dtype == "BF16":
            a = (a.view(np.uint32) >> 16).astype(np.uint16)  # exact for the bf16-representable values used
        out[name] = (dtype, a.reshape(shape) if shape else a)

    pre = "language_model.model"
    affine(pre + ".embed_tokens", -1, K_EMBED, cfg.vocab, H)
    affine("language_model.lm_head", -1, K_HEAD, cfg.vocab, H)
    vec(pre + ".norm.weight", -1, K_FINAL_NORM, H, "BF16")
    for i in range(cfg.n_layers):
        p = f"{pre}.layers.{i}"
        vec(p + ".input_layernorm.weight", i, K_IN_NORM, H, "BF16")
        vec(p + ".post_attention_layernorm.weight", i, K_POST_NORM, H, "BF16")
        affine(p + ".mlp.gate_proj", i, K_GATE, cfg.intermediate, H)
        affine(p + ".mlp.up_proj", i, K_UP, cfg.intermediate, H)
        affine(p + ".mlp.down_proj", i, K_DOWN, H, cfg.intermediate)
        if i % cfg.full_every == cfg.full_every - 1:
            affine(p + ".self_attn.q_proj", i, K_Q, 2 * cfg.heads * cfg.head_dim, H)
            affine(p + ".self_attn.k_proj", i, K_K, cfg.kv_heads * cfg.head_dim, H)
            affine(p + ".self_attn.v_proj", i, K_V, cfg.kv_heads * cfg.head_dim, H)
            affine(p + ".self_attn.o_proj", i, K_O, H, cfg.heads * cfg.head_dim)
            vec(p + ".self_attn.q_norm.weight", i, K_QNORM, cfg.head_dim, "BF16")
            vec(p + ".self_attn.k_norm.weight", i, K_KNORM, cfg.head_dim, "F32")
        else:
            affine(p + ".linear_attn.in_proj_qkv", i, K_QKV, conv_dim, H)
            affine(p + ".linear_attn.in_proj_z", i, K_Z, value_dim, H)
            affine(p + ".linear_attn.in_proj_a", i, K_A, cfg.v_heads, H)
            affine(p + ".linear_attn.in_proj_b", i, K_B, cfg.v_heads, H)
            affine(p + ".linear_attn.out_proj", i, K_OUT, H, value_dim)
            vec(p + ".linear_attn.conv1d.weight", i, K_CONV, conv_dim * cfg.conv_kernel, "F32",
                (conv_dim, cfg.conv_kernel, 1))
            vec(p + ".linear_attn.A_log", i, K_ALOG, cfg.v_heads)
            vec(p + ".linear_attn.dt_bias", i, K_DTB, cfg.v_heads)
            vec(p + ".linear_attn.norm.weight", i, K_GNORM, cfg.v_dim, "BF16")
    return out


def perturb_norms_qwen35(cfg, oracle, rng) -> None:
    """Give every norm weight of the oracle model distinct bf16-exact values
    in [0.5, 1.5), so a loader that swaps two norms changes the logits."""
    def set_vec(layer, kind, n):
        a = host_array(oracle.tensor_ptr(layer, kind), C.c_float, n)
        v = rng.uniform(0.5, 1.5, n).astype(np.float32)
        a[:] = ((v.view(np.uint32) >> 16) << 16).view(np.float32)

    set_vec(-1, K_FINAL_NORM, cfg.hidden)
    for i in range(cfg.n_layers):
        set_vec(i, K_IN_NORM, cfg.hidden)
        set_vec(i, K_POST_NORM, cfg.hidden)
        if i % cfg.full_every == cfg.full_every - 1:
            set_vec(i, K_QNORM, cfg.head_dim)
            set_vec(i, K_KNORM, cfg.head_dim)
        else:
            set_vec(i, K_GNORM, cfg.v_dim)


# ---------------------------------------------------------------------------
# GGUF
# ---------------------------------------------------------------------------
G_U32, G_I32, G_F32, G_STR, G_ARR = 4, 5, 6, 8, 9
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q5_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 2, 6, 8, 12, 14


def _gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _gval(t: int, v) -> bytes:
    if t == G_U32:
        return struct.pack("<I", v)
    if t == G_I32:
        return struct.pack("<i", v)
    if t == G_F32:
        return struct.pack("<f", v)
    if t == G_STR:
        return _gstr(v)
    if t == G_ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_gval(et, x) for x in items)
    raise ValueError(t)


def write_gguf(path: Path, meta: list, tensors: list, align: int = 32) -> None:
    """meta: [(key, type, value)]; tensors: [(name, ggml_type, ne (innermost
    first), raw bytes)]."""
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta))
    for k, t, v in meta:
        head += _gstr(k) + struct.pack("<I", t) + _gval(t, v)
    data = b""
    infos = b""
    for name, gt, ne, raw in tensors:
        off = (len(data) + align - 1) // align * align
        data += b"\0" * (off - len(data)) + raw
        infos += _gstr(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        infos += struct.pack("<IQ", gt, off)
    head += infos
    pad = (len(head) + align - 1) // align * align - len(head)
    path.write_bytes(head + b"\0" * pad + data)


def qwen2_meta(cfg, arch="qwen2") -> list:
    return [("general.architecture", G_STR, arch),
            ("general.alignment", G_U32, 32),
            ("qwen2.block_count", G_U32, cfg.n_layers),
            ("qwen2.context_length", G_U32, cfg.max_pos),
            ("qwen2.embedding_length", G_U32, cfg.hidden),
            ("qwen2.feed_forward_length", G_U32, cfg.intermediate),
            ("qwen2.attention.head_count", G_U32, cfg.heads),
            ("qwen2.attention.head_count_kv", G_U32, cfg.kv_heads),
            ("qwen2.rope.freq_base", G_F32, cfg.rope_theta),
            ("qwen2.attention.layer_norm_rms_epsilon", G_F32, cfg.eps),
            # tokenizer tables are skipped by the reader
            ("tokenizer.ggml.tokens", G_ARR, (G_STR, ["a", "bc", "<|x|>"])),
            ("tokenizer.ggml.token_type", G_ARR, (G_I32, [1, 1, 3]))]


BLOCK_BYTES = {GGML_Q4_K: (256, 144), GGML_Q6_K: (256, 210), GGML_Q8_0: (32, 34), GGML_Q5_0: (32, 22)}
ORACLE_FMT = {GGML_Q4_K: 1, GGML_Q6_K: 2, GGML_Q8_0: 3, GGML_Q5_0: 4}


def gguf_tensors_from_oracle(cfg, oracle, untied: bool = False, types=None) -> list:
    """Qwen2 tensors as the oracle holds them: by default its synthetic
    formats (Q6_K embedding, attn_v and even ffn_down; Q4_K elsewhere);
    types[(layer, kind)] names another ggml type for a matrix the oracle
    holds in that type (ora.Qwen2.set_matrix). Norms and biases F32."""
    H, kvw = cfg.hidden, cfg.kv_heads * cfg.head_dim
    types = types or {}
    out = []

    def mat(name, layer, kind, n_out, n_in, q6):
        gt = types.get((layer, kind), GGML_Q6_K if q6 else GGML_Q4_K)
        per, nbytes = BLOCK_BYTES[gt]
        raw = host_array(oracle.tensor_ptr(layer, kind), C.c_uint8, n_out * (n_in // per) * nbytes).tobytes()
        out.append((name, gt, (n_in, n_out), raw))

    def vec(name, layer, kind, n):
        out.append((name, GGML_F32, (n,), host_array(oracle.tensor_ptr(layer, kind), C.c_float, n).tobytes()))

    mat("token_embd.weight", -1, K_EMBED, cfg.vocab, H, True)
    if untied:
        mat("output.weight", -1, K_EMBED, cfg.vocab, H, True)
    vec("output_norm.weight", -1, K_FINAL_NORM, H)
    for i in range(cfg.n_layers):
        p = f"blk.{i}"
        vec(p + ".attn_norm.weight", i, K_IN_NORM, H)
        vec(p + ".ffn_norm.weight", i, K_POST_NORM, H)
        mat(p + ".attn_q.weight", i, K_Q, cfg.heads * cfg.head_dim, H, False)
        mat(p + ".attn_k.weight", i, K_K, kvw, H, False)
        mat(p + ".attn_v.weight", i, K_V, kvw, H, True)
        mat(p + ".attn_output.weight", i, K_O, H, cfg.heads * cfg.head_dim, False)
        vec(p + ".attn_q.bias", i, K_QB, cfg.heads * cfg.head_dim)
        vec(p + ".attn_k.bias", i, K_KB, kvw)
        vec(p + ".attn_v.bias", i, K_VB, kvw)
        mat(p + ".ffn_gate.weight", i, K_GATE, cfg.intermediate, H, False)
        mat(p + ".ffn_up.weight", i, K_UP, cfg.intermediate, H, False)
        mat(p + ".ffn_down.weight", i, K_DOWN, H, cfg.intermediate, i % 2 == 0)
    return out


def random_blocks(rng, ggml_type: int, n_out: int, n_in: int, d_std: float = 5e-4) -> np.ndarray:
    """Random Q8_0 / Q5_0 blocks: f16 scales N(0, d_std), uniform quants."""
    nb = n_out * n_in // 32
    d = rng.normal(0, d_std, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    if ggml_type == GGML_Q8_0:
        q = rng.integers(0, 256, (nb, 32), dtype=np.uint8)
        return np.concatenate([d, q], axis=1).reshape(-1)
    qh = rng.integers(0, 256, (nb, 4), dtype=np.uint8)
    qs = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    return np.concatenate([d, qh, qs], axis=1).reshape(-1)


def perturb_norms_qwen2(cfg, oracle, rng) -> None:
    def set_vec(layer, kind, n):
        host_array(oracle.tensor_ptr(layer, kind), C.c_float, n)[:] = rng.uniform(0.5, 1.5, n).astype(np.float32)

    set_vec(-1, K_FINAL_NORM, cfg.hidden)
    for i in range(cfg.n_layers):
        set_vec(i, K_IN_NORM, cfg.hidden)
        set_vec(i, K_POST_NORM, cfg.hidden)
