"""Pins the oracle's cache bytes v1 (pagoda-hf/src/qwen3_5.rs:177-256): the
reference's own round-trip fixture spelled out byte for byte, the reader's
error cases, and the layouts inside a model-written cache (conv history
[conv_dim, kernel-1] oldest first, recurrent state [v_heads, k_dim, v_dim],
KV [len, kv_heads, head_dim]) through properties of the recurrence that a
transposed or reordered layout fails."""
import numpy as np
import pytest

from oracle import pyoracle as ora
import cachev1

# qwen3_5.rs:1909-1948 kv_host_bytes_roundtrip: len 2; layer 0 linear with
# conv [1, 2], state [3]; layer 1 full with k [4..7], v [8..11], kv_heads 1,
# head_dim 2.
FIXTURE = bytes.fromhex(
    "01000000"                      # version 1
    "0200000000000000"              # len 2 (u64)
    "02000000"                      # 2 layers
    "01"                            # linear
    "02000000" "0000803f" "00000040"  # conv [1, 2]
    "01000000" "00004040"             # state [3]
    "02"                            # full
    "02000000" "01000000" "02000000"  # kv_len 2, kv_heads 1, head_dim 2
    "04000000" "00008040" "0000a040" "0000c040" "0000e040"  # k [4..7]
    "04000000" "00000041" "00001041" "00002041" "00003041"  # v [8..11]
)


def test_reference_fixture_round_trips_byte_exact():
    c = ora.Qwen35Cache.from_bytes(FIXTURE)
    assert len(c) == 2
    assert c.to_bytes() == FIXTURE


def test_reader_reads_reference_fixture():
    p = cachev1.parse(FIXTURE)
    assert p["len"] == 2 and [L["tag"] for L in p["layers"]] == [1, 2]
    np.testing.assert_array_equal(p["layers"][0]["conv"], [1, 2])
    np.testing.assert_array_equal(p["layers"][0]["state"], [3])
    L = p["layers"][1]
    assert (L["kv_len"], L["kv_heads"], L["head_dim"]) == (2, 1, 2)
    np.testing.assert_array_equal(L["k"], [4, 5, 6, 7])
    np.testing.assert_array_equal(L["v"], [8, 9, 10, 11])


@pytest.mark.parametrize("bad", [
    b"\x02" + FIXTURE[1:],                          # version 2
    FIXTURE[:16] + b"\x03" + FIXTURE[17:],          # unknown tag
    FIXTURE + b"\x00",                              # trailing byte
    FIXTURE[:-1],                                   # truncated
    FIXTURE[:42] + b"\x03\x00\x00\x00" + FIXTURE[46:],  # kv_len 3: k/v count mismatch
    b"",
])
def test_malformed_bytes_rejected(bad):
    with pytest.raises(ValueError):
        ora.Qwen35Cache.from_bytes(bad)
    with pytest.raises(ValueError):
        cachev1.parse(bad)


def _tiny():
    cfg = ora.Qwen35Config(n_layers=4, hidden=128, intermediate=256, vocab=512, heads=2, kv_heads=2, head_dim=64,
                           rotary_dim=16, rope_theta=1e7, k_heads=2, v_heads=4, k_dim=32, v_dim=32,
                           conv_kernel=4, full_every=4)
    return cfg, ora.Qwen35(cfg, 5)


def test_model_cache_layouts():
    cfg, m = _tiny()
    conv_dim = 2 * cfg.k_heads * cfg.k_dim + cfg.v_heads * cfg.v_dim
    c1 = m.new_cache()
    m.forward([7], c1)
    c2 = c1.clone()
    m.forward([9], c2)
    p1, p2 = cachev1.parse(c1.to_bytes()), cachev1.parse(c2.to_bytes())
    assert p1["len"] == 1 and p2["len"] == 2
    assert [L["tag"] for L in p1["layers"]] == [1, 1, 1, 2]
    for L1, L2 in zip(p1["layers"][:3], p2["layers"][:3]):
        # conv history [conv_dim, 3], oldest first: after one token only the
        # newest column is set; the next token shifts it one column left
        h1 = L1["conv"].reshape(conv_dim, 3)
        h2 = L2["conv"].reshape(conv_dim, 3)
        assert not h1[:, :2].any() and h1[:, 2].any()
        np.testing.assert_array_equal(h2[:, 1], h1[:, 2])
        assert not h2[:, 0].any()
        # from S = 0 one step gives S[h] = k_h delta_h^T (rank one, k along
        # the k_dim axis); value heads 2j and 2j+1 share key head j, so their
        # states share the left singular vector, not the right one
        S = L1["state"].reshape(cfg.v_heads, cfg.k_dim, cfg.v_dim).astype(np.float64)
        for j in range(cfg.k_heads):
            u = [np.linalg.svd(S[2 * j + r])[0][:, 0] for r in range(2)]
            w = [np.linalg.svd(S[2 * j + r])[2][0] for r in range(2)]
            sv = np.linalg.svd(S[2 * j], compute_uv=False)
            assert sv[1] < 1e-5 * sv[0]
            assert abs(u[0] @ u[1]) > 1 - 1e-6
            assert abs(w[0] @ w[1]) < 0.9
            # k is L2-normalized: the column space vector is k itself
    # KV [len, kv_heads, head_dim]: the one-token cache is a prefix of the
    # two-token one, and each (position, head) row after the k RMSNorm (unit
    # weight) and the norm-preserving RoPE has mean square 1
    k1, k2 = p1["layers"][3]["k"], p2["layers"][3]["k"]
    w = cfg.kv_heads * cfg.head_dim
    np.testing.assert_array_equal(k2[:w], k1)
    np.testing.assert_array_equal(p2["layers"][3]["v"][:w], p1["layers"][3]["v"])
    ms = (k2.astype(np.float64).reshape(2, cfg.kv_heads, cfg.head_dim) ** 2).mean(-1)
    np.testing.assert_allclose(ms, 1.0, rtol=1e-4)


def test_from_bytes_continues_like_the_cache():
    _, m = _tiny()
    c = m.new_cache()
    m.forward([3, 1, 4, 1, 5], c)
    d = ora.Qwen35Cache.from_bytes(c.to_bytes(), m)
    assert d.to_bytes() == c.to_bytes()
    a = m.forward([9, 2], c)
    b = m.forward([9, 2], d)
    np.testing.assert_array_equal(a, b)
    assert d.to_bytes() == c.to_bytes()
