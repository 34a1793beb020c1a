"""Checkpoint readers without a device: the configuration pgd_checkpoint_config
derives from an MLX directory (qwen3_5.rs:338-383) or a Qwen2 GGUF file
(qwen2_gguf.rs:65-91), and the format errors both report."""
import json
import struct

import numpy as np
import pytest

from checkpoints import (G_F32, G_STR, G_U32, GGML_F32, GGML_Q4_0, GGML_Q4_K, GGML_Q6_K, mlx_text_config,
                         qwen2_meta, write_gguf, write_mlx_config, write_safetensors_shards)


def cfgs():
    from pagoda_amd.engine import ARCH_QWEN2, ModelConfig

    q35 = ModelConfig(n_layers=8, hidden=256, intermediate=512, vocab=1024, heads=4, kv_heads=2, head_dim=128,
                      rotary_dim=32, rope_theta=1e7, eps=1e-6, k_heads=2, v_heads=4, k_dim=128, v_dim=128,
                      conv_kernel=4, full_every=4, max_pos=4096, kv_block=16, kv_blocks=64)
    q2 = ModelConfig(arch=ARCH_QWEN2, n_layers=2, hidden=256, intermediate=512, vocab=1000, heads=4, kv_heads=2,
                     head_dim=64, rotary_dim=64, rope_theta=1e6, eps=1e-6, k_heads=0, v_heads=0, k_dim=0, v_dim=0,
                     conv_kernel=0, full_every=1, max_pos=2048, kv_block=16, kv_blocks=64)
    return q35, q2


def same_config(a, b):
    """Equal field by field; float fields at the C struct's float32 precision."""
    from dataclasses import asdict

    da, db = asdict(a), asdict(b)
    for k in da:
        if isinstance(da[k], float) or isinstance(db[k], float):
            assert np.float32(da[k]) == np.float32(db[k]), k
        else:
            assert da[k] == db[k], k


def mlx_dir(tmp_path, text=None, quant=None, embed_shape=None):
    q35, _ = cfgs()
    d = tmp_path / "mlx"
    write_mlx_config(d, text or mlx_text_config(q35, max_pos=q35.max_pos), quant)
    rows, cols = embed_shape or (q35.vocab, q35.hidden // 4)
    write_safetensors_shards(d, {
        "language_model.model.embed_tokens.weight": ("U32", np.zeros((rows, cols), np.uint32)),
        "language_model.model.embed_tokens.scales": ("BF16", np.zeros((rows, 4), np.uint16)),
        "language_model.model.norm.weight": ("F32", np.ones(q35.hidden, np.float32))})
    return d


def config(path, max_pos=0, kv_blocks=64):
    from pagoda_amd.engine import checkpoint_config

    return checkpoint_config(str(path), max_pos, kv_blocks)


def expect_error(path, fragment, code=-7, **kw):
    from pagoda_amd._lib import PagodaError

    with pytest.raises(PagodaError) as e:
        config(path, **kw)
    assert e.value.code == code
    assert fragment in str(e.value), str(e.value)


def test_mlx_config_matches_the_model_config(tmp_path):
    q35, _ = cfgs()
    same_config(config(mlx_dir(tmp_path)), q35)
    # an explicit max_pos wins over max_position_embeddings
    assert config(mlx_dir(tmp_path), max_pos=777).max_pos == 777


def test_mlx_irregular_layer_pattern(tmp_path):
    q35, _ = cfgs()
    kinds = ["linear_attention", "full_attention"] + ["linear_attention"] * 5 + ["full_attention"]
    got = config(mlx_dir(tmp_path, text=mlx_text_config(q35, max_pos=64, layer_types=kinds)))
    assert got.full_every == 0 and got.n_layers == 8


@pytest.mark.parametrize("mutate,fragment", [
    (lambda t, q: q.update(bits=4), "8-bit"),
    (lambda t, q: q.update(group_size=32), "group size 64"),
    (lambda t, q: q.update(mode="mxfp4"), "affine"),
    (lambda t, q: t["layer_types"].__setitem__(0, "sliding_attention"), "unknown layer type sliding_attention"),
    (lambda t, q: t["layer_types"].pop(), "layer_types length"),
    (lambda t, q: t.pop("head_dim"), "head_dim"),
    (lambda t, q: t.pop("max_position_embeddings"), "max_pos"),
])
def test_mlx_config_errors(tmp_path, mutate, fragment):
    q35, _ = cfgs()
    text = mlx_text_config(q35, max_pos=q35.max_pos)
    quant = {"bits": 8, "group_size": 64, "mode": "affine"}
    mutate(text, quant)
    expect_error(mlx_dir(tmp_path, text=text, quant=quant), fragment)


def test_mlx_store_errors(tmp_path):
    # embedding shape disagrees with the config
    expect_error(mlx_dir(tmp_path, embed_shape=(1000, 64)), "embed_tokens")
    # kv_blocks must be given
    expect_error(mlx_dir(tmp_path), "kv_blocks", code=-1, kv_blocks=0)
    # a shard whose header length runs past the end of the file
    d = mlx_dir(tmp_path)
    shard = sorted(d.glob("*.safetensors"))[0]
    raw = bytearray(shard.read_bytes())
    raw[:8] = struct.pack("<Q", len(raw))
    shard.write_bytes(bytes(raw))
    expect_error(d, "header length")
    # malformed config.json
    (d / "config.json").write_text("{\"text_config\": [1, 2,}")
    expect_error(d, "json")


def gguf_file(tmp_path, meta=None, emb_type=GGML_Q6_K, emb_ne=None, corrupt=None):
    _, q2 = cfgs()
    emb_ne = emb_ne or (q2.hidden, q2.vocab)
    nb = emb_ne[1] * (emb_ne[0] // 256)
    emb_bytes = {GGML_Q6_K: 210 * nb, GGML_Q4_K: 144 * nb, GGML_Q4_0: 18 * emb_ne[1] * (emb_ne[0] // 32)}[emb_type]
    tensors = [("token_embd.weight", emb_type, emb_ne, bytes(emb_bytes)),
               ("output_norm.weight", GGML_F32, (q2.hidden,), np.ones(q2.hidden, np.float32).tobytes()),
               ("blk.0.ffn_gate.weight", GGML_Q4_K, (q2.hidden, q2.intermediate),
                bytes(144 * q2.intermediate * (q2.hidden // 256)))]
    p = tmp_path / "m.gguf"
    write_gguf(p, meta if meta is not None else qwen2_meta(q2), tensors)
    if corrupt:
        p.write_bytes(corrupt(p.read_bytes()))
    return p


def test_gguf_config_matches_the_model_config(tmp_path):
    _, q2 = cfgs()
    same_config(config(gguf_file(tmp_path)), q2)


def test_gguf_config_defaults(tmp_path):
    _, q2 = cfgs()
    # no rope.freq_base: 1e6 (qwen2_gguf.rs:78-82); no feed_forward_length: ffn_gate rows
    meta = [m for m in qwen2_meta(q2) if m[0] not in ("qwen2.rope.freq_base", "qwen2.feed_forward_length")]
    got = config(gguf_file(tmp_path, meta=meta), max_pos=100)
    assert got.rope_theta == np.float32(1e6) and got.intermediate == q2.intermediate and got.max_pos == 100


@pytest.mark.parametrize("case,fragment", [
    ("arch", "only Qwen2 GGUF"),
    ("magic", "not a GGUF file"),
    ("version", "GGUF version 1"),
    ("truncated", "truncated"),
    ("q4_0", "token_embd.weight has ggml type 2"),
    ("ragged", "super-blocks"),
    ("range", "out of range"),
    ("heads", "head_count_kv"),
])
def test_gguf_errors(tmp_path, case, fragment):
    _, q2 = cfgs()
    meta = qwen2_meta(q2)
    kw = {}
    if case == "arch":
        kw["meta"] = [("general.architecture", G_STR, "llama")] + meta[1:]
    elif case == "magic":
        kw["corrupt"] = lambda b: b"GGUX" + b[4:]
    elif case == "version":
        kw["corrupt"] = lambda b: b[:4] + struct.pack("<I", 1) + b[8:]
    elif case == "truncated":
        kw["corrupt"] = lambda b: b[:200]
    elif case == "q4_0":
        kw["emb_type"] = GGML_Q4_0
    elif case == "ragged":
        kw["emb_type"], kw["emb_ne"] = GGML_Q4_K, (96, q2.vocab)
    elif case == "range":
        kw["corrupt"] = lambda b: b[:-1000]
    elif case == "heads":
        kw["meta"] = [m for m in meta if m[0] != "qwen2.attention.head_count_kv"]
    expect_error(gguf_file(tmp_path, **kw), fragment)


def test_gguf_huge_dims_are_rejected(tmp_path):
    """Dimensions whose product overflows 64-bit byte counts must not pass
    the bounds check."""
    _, q2 = cfgs()
    p = tmp_path / "huge.gguf"
    write_gguf(p, qwen2_meta(q2), [("token_embd.weight", GGML_Q4_K, (256, 1 << 62), bytes(144))])
    expect_error(p, "too large")


def test_safetensors_huge_shape_is_rejected(tmp_path):
    d = mlx_dir(tmp_path)
    shard = sorted(d.glob("*.safetensors"))[0]
    raw = shard.read_bytes()
    n = int.from_bytes(raw[:8], "little")
    hdr = json.loads(raw[8:8 + n])
    name = next(k for k in hdr if k != "__metadata__")
    hdr[name]["shape"] = [1 << 40, 1 << 40]
    h = json.dumps(hdr).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    shard.write_bytes(len(h).to_bytes(8, "little") + h + raw[8 + n:])
    expect_error(d, "too large")
