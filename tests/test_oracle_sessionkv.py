"""Pins the oracle's SessionKv PD payload (pagoda-hf/src/llama.rs:215-345):
the reference's own round-trip assertions (llama.rs:352-450: f16 exact and
tolerant values, byte counts of the f16 wire, logits kept f32-exact, corrupt
payloads rejected), the [kv_heads, len, head_dim] tensor order through the
per-head prefix property, and that an imported cache continues bitwise like
the one exported."""
import numpy as np
import pytest

import sessionkv
from oracle import pyoracle as ora


def tiny():
    cfg = ora.Qwen2Config(n_layers=3, hidden=256, intermediate=512, vocab=512, heads=4, kv_heads=2, head_dim=64,
                          max_pos=256, rope_theta=1e6, eps=1e-6)
    return ora.Qwen2(cfg, 3)


def test_f16_wire_values_of_reference_test():
    # llama.rs:352-365
    for x in [0.0, 1.0, -1.0, 0.5, -0.5, 65504.0, -65504.0]:
        assert ora.f16_to_f32(ora.f32_to_f16(x)) == x
    for x in [0.1, 0.3333, 100.25, -1234.5]:
        back = ora.f16_to_f32(ora.f32_to_f16(x))
        assert abs(back - np.float32(x)) <= abs(x) * 0.001 + 1e-6
    assert ora.f16_to_f32(ora.f32_to_f16(np.inf)) == np.inf
    assert np.isnan(ora.f16_to_f32(ora.f32_to_f16(np.nan)))


def test_export_layout_and_round_trip():
    m = tiny()
    cfg = m.cfg
    prompt = [5, 17, 33, 2, 9]
    c = m.new_cache()
    logits = m.forward(prompt, c)
    blob = c.export_bytes(logits)
    p = sessionkv.parse(blob)
    assert p["version"] == 2 and p["len"] == 5 and len(p["layers"]) == cfg.n_layers and p["trailing"] == 0
    np.testing.assert_array_equal(p["logits"], logits)
    for L in p["layers"]:
        assert (L["kv_heads"], L["head_dim"], L["dtype"]) == (cfg.kv_heads, cfg.head_dim, 0)
    # [kv_heads, len, head_dim]: each head's rows of the 5-token cache are a
    # prefix of that head's rows after one more token
    d = ora.Qwen2Cache.import_bytes(m, blob)[0]
    m.forward([11], d)
    q = sessionkv.parse(d.export_bytes())
    for L, M in zip(p["layers"], q["layers"]):
        np.testing.assert_array_equal(M["k"][:, :5], L["k"])
        np.testing.assert_array_equal(M["v"][:, :5], L["v"])
    # the payload re-exports byte for byte and continues like the original
    e, lg = ora.Qwen2Cache.import_bytes(m, blob)
    np.testing.assert_array_equal(lg, logits)
    assert e.export_bytes(lg) == blob
    np.testing.assert_array_equal(m.forward([11, 4], e), m.forward([11, 4], c))


def test_f16_wire_byte_count_and_values():
    """llama.rs:367-398: the f16 wire saves 2 bytes per K/V value; logits stay f32-exact."""
    m = tiny()
    cfg = m.cfg
    c = m.new_cache()
    logits = m.forward([1, 2, 3, 4, 5], c)
    b32, b16 = c.export_bytes(logits), c.export_bytes(logits, f16=True)
    assert len(b16) == len(b32) - cfg.n_layers * cfg.kv_heads * 5 * cfg.head_dim * 2 * 2
    p32, p16 = sessionkv.parse(b32), sessionkv.parse(b16)
    np.testing.assert_array_equal(p16["logits"], logits)
    for L32, L16 in zip(p32["layers"], p16["layers"]):
        assert L16["dtype"] == 1
        np.testing.assert_array_equal(L16["k"], L32["k"].astype(np.float16))  # numpy as the independent codec
        np.testing.assert_array_equal(L16["v"], L32["v"].astype(np.float16))
    e, lg = ora.Qwen2Cache.import_bytes(m, b16)
    np.testing.assert_array_equal(lg, logits)
    q = sessionkv.parse(e.export_bytes())
    for L, M in zip(p16["layers"], q["layers"]):
        np.testing.assert_array_equal(M["k"], L["k"].astype(np.float32))


def test_hand_written_payload_imports():
    m = tiny()
    cfg = m.cfg
    rng = np.random.default_rng(1)
    layers = [(rng.random((cfg.kv_heads, 5, cfg.head_dim), np.float32),
               rng.random((cfg.kv_heads, 5, cfg.head_dim), np.float32)) for _ in range(cfg.n_layers)]
    for version in (1, 2):
        blob = sessionkv.write(5, layers, logits=[0.25, -1.5, 3.75], version=version)
        c, lg = ora.Qwen2Cache.import_bytes(m, blob)
        assert len(c) == 5
        np.testing.assert_array_equal(lg, np.float32([0.25, -1.5, 3.75]))
        p = sessionkv.parse(c.export_bytes(lg))
        for (k, v), L in zip(layers, p["layers"]):
            np.testing.assert_array_equal(L["k"], k)
            np.testing.assert_array_equal(L["v"], v)
    # version 1: the dtype field is informational, the payload is f32
    blob = bytearray(sessionkv.write(5, layers, version=1))
    c, lg = ora.Qwen2Cache.import_bytes(m, bytes(blob))
    assert lg is None and len(c) == 5


@pytest.mark.parametrize("cut", ["12", "garbage", "magic", "version", "heads", "short"])
def test_corrupt_payloads_fail(cut):
    m = tiny()
    cfg = m.cfg
    c = m.new_cache()
    m.forward([1, 2, 3], c)
    blob = c.export_bytes()
    bad = {"12": blob[:12], "garbage": b"garbage", "magic": b"\0" + blob[1:],
           "version": blob[:4] + b"\x03" + blob[5:], "short": blob[:-1],
           "heads": sessionkv.write(3, [(np.zeros((1, 3, cfg.head_dim)),) * 2] * cfg.n_layers)}[cut]
    with pytest.raises(ValueError):
        ora.Qwen2Cache.import_bytes(m, bad)
