"""Pins the oracle's Gated-DeltaNet, attention, conv and RoPE restatements
with closed forms and invariants (independent of the code under test)."""
import numpy as np
import pytest

from oracle import pyoracle as ora


def l2n(x):
    return x / np.sqrt((x * x).sum() + 1e-6)


def gates(rng, vh):
    return rng.normal(0, 1, vh).astype(np.float32), rng.normal(0, 1, vh).astype(np.float32)


def make_inputs(rng, kh, vh, d, seq):
    conv = rng.normal(0, 1, (seq, 2 * kh * d + vh * d)).astype(np.float32)
    a = rng.normal(0, 1, (seq, vh)).astype(np.float32)
    b = rng.normal(0, 1, (seq, vh)).astype(np.float32)
    z = rng.normal(0, 1, (seq, vh * d)).astype(np.float32)
    return conv, a, b, z


def softplus(x):
    return np.log1p(np.exp(x))


def test_gdn_single_step_from_zero_closed_form():
    """From S = 0: S' = k (beta v)^T, so o = S'^T q = beta (q.k) v, then the
    gated RMSNorm o * rsqrt(mean o^2 + eps) * w * silu(z)."""
    rng = np.random.default_rng(0)
    kh, vh, d = 2, 4, 128
    conv, a, b, z = make_inputs(rng, kh, vh, d, 1)
    a_log = rng.uniform(0, 2.7, vh).astype(np.float32)
    dtb = rng.normal(0, 0.1, vh).astype(np.float32)
    norm = rng.uniform(0.5, 1.5, d).astype(np.float32)
    state = np.zeros((vh, d, d), np.float32)
    out = ora.gdn_step(conv, a, b, z, a_log, dtb, norm, kh, vh, d, d, state)
    q = conv[0, :kh * d].reshape(kh, d)
    k = conv[0, kh * d:2 * kh * d].reshape(kh, d)
    v = conv[0, 2 * kh * d:].reshape(vh, d)
    for h in range(vh):
        qq = l2n(q[h // 2].astype(np.float64)) / np.sqrt(d)
        kk = l2n(k[h // 2].astype(np.float64))
        beta = 1 / (1 + np.exp(-b[0, h]))
        o = beta * (qq @ kk) * v[h]
        o = o / np.sqrt((o * o).mean() + 1e-6) * norm * (z[0, h * d:(h + 1) * d] / (1 + np.exp(-z[0, h * d:(h + 1) * d])))
        np.testing.assert_allclose(out[0, h * d:(h + 1) * d], o, rtol=2e-4, atol=1e-6)
        np.testing.assert_allclose(state[h], np.outer(kk, beta * v[h]), rtol=2e-4, atol=1e-7)


def test_gdn_beta_zero_only_decays():
    rng = np.random.default_rng(1)
    kh, vh, d = 1, 2, 128
    conv, a, b, z = make_inputs(rng, kh, vh, d, 1)
    b[:] = -200.0  # sigmoid -> 0
    a_log = np.array([0.7, 1.9], np.float32)
    dtb = np.array([0.2, -0.3], np.float32)
    s0 = rng.normal(0, 1, (vh, d, d)).astype(np.float32)
    state = s0.copy()
    ora.gdn_step(conv, a, b, z, a_log, dtb, np.ones(d, np.float32), kh, vh, d, d, state)
    for h in range(vh):
        decay = np.exp(-np.exp(a_log[h]) * softplus(a[0, h] + dtb[h]))
        np.testing.assert_allclose(state[h], s0[h] * decay, rtol=1e-5, atol=1e-7)


def test_gdn_delta_rule_stores_value():
    """decay = 1 and beta = 1 with a unit key: after the update S^T k == v."""
    rng = np.random.default_rng(2)
    kh, vh, d = 1, 1, 128
    conv, a, b, z = make_inputs(rng, kh, vh, d, 1)
    a[:] = -100.0  # softplus -> ~0, decay -> 1
    b[:] = 100.0   # beta -> 1
    state = rng.normal(0, 0.1, (vh, d, d)).astype(np.float32)
    ora.gdn_step(conv, a, b, z, np.zeros(1, np.float32), np.zeros(1, np.float32), np.ones(d, np.float32),
                 kh, vh, d, d, state)
    k = l2n(conv[0, d:2 * d].astype(np.float64))
    v = conv[0, 2 * d:]
    np.testing.assert_allclose(state[0].T.astype(np.float64) @ k, v, rtol=1e-4, atol=1e-4)


def test_gdn_chunk_equals_sequential_steps():
    rng = np.random.default_rng(3)
    kh, vh, d, seq = 2, 4, 128, 4
    conv, a, b, z = make_inputs(rng, kh, vh, d, seq)
    a_log = rng.uniform(0, 2.7, vh).astype(np.float32)
    dtb = rng.normal(0, 0.1, vh).astype(np.float32)
    norm = np.ones(d, np.float32)
    s1 = rng.normal(0, 0.1, (vh, d, d)).astype(np.float32)
    s2 = s1.copy()
    chunk = ora.gdn_step(conv, a, b, z, a_log, dtb, norm, kh, vh, d, d, s1)
    seq_out = np.concatenate([ora.gdn_step(conv[t:t + 1], a[t:t + 1], b[t:t + 1], z[t:t + 1], a_log, dtb, norm,
                                           kh, vh, d, d, s2) for t in range(seq)])
    np.testing.assert_array_equal(chunk, seq_out)
    np.testing.assert_array_equal(s1, s2)


def test_attention_matches_textbook_two_pass():
    rng = np.random.default_rng(4)
    heads, kvh, hd, n = 6, 2, 64, 37
    q = rng.normal(0, 1, (heads, hd)).astype(np.float32)
    k = rng.normal(0, 1, (n, kvh, hd)).astype(np.float32)
    v = rng.normal(0, 1, (n, kvh, hd)).astype(np.float32)
    g = rng.normal(0, 1, (heads, hd)).astype(np.float32)
    out = ora.attn_decode(q, k, v, n, heads, kvh, hd, g)
    for h in range(heads):
        kk = k[:, h // 3].astype(np.float64)
        s = kk @ q[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        o = p @ v[:, h // 3] / (1 + np.exp(-g[h].astype(np.float64)))
        np.testing.assert_allclose(out[h], o, rtol=1e-4, atol=1e-6)
    # one position: output is exactly that value row (softmax of one score)
    out1 = ora.attn_decode(q, k, v, 1, heads, kvh, hd)
    np.testing.assert_allclose(out1, v[0][np.arange(heads) // 3], rtol=1e-6)


@pytest.mark.parametrize("seq", [1, 2, 3, 5])
def test_causal_conv_matches_direct_definition(seq):
    rng = np.random.default_rng(5 + seq)
    ch, K = 10, 4
    x = rng.normal(0, 1, (seq, ch)).astype(np.float32)
    w = rng.normal(0, 0.3, (ch, K)).astype(np.float32)
    st = rng.normal(0, 1, (ch, K - 1)).astype(np.float32)
    full = np.concatenate([st.T, x], 0)  # [K-1+seq, ch]
    exp = np.zeros((seq, ch))
    for t in range(seq):
        win = full[t:t + K]  # oldest first
        acc = (win * w.T).sum(0)
        exp[t] = acc / (1 + np.exp(-acc))
    st2 = st.copy()
    out = ora.causal_conv(x, K, w, st2)
    np.testing.assert_allclose(out, exp, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(st2, full[-(K - 1):].T)


def test_rope_tables_and_rotation():
    c, s = ora.rope_cos_sin(0, 64, 1e7)
    np.testing.assert_array_equal(c, np.ones(64, np.float32))
    np.testing.assert_array_equal(s, np.zeros(64, np.float32))
    c, s = ora.rope_cos_sin(5, 64, 1e7)
    freq = 1.0 / np.power(1e7, np.arange(0, 64, 2) / 64.0)
    np.testing.assert_allclose(c[:32], np.cos(5 * freq), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(c[32:], c[:32])
    np.testing.assert_allclose(s[:32], np.sin(5 * freq), rtol=1e-5, atol=1e-6)


def test_argmax_first_tie_rule():
    x = np.array([1.0, 3.0, np.nan, 3.0, np.inf, -1.0], np.float32)
    assert ora.argmax_first(x) == 1
    assert ora.argmax_first(np.array([np.nan, np.inf], np.float32)) == 0


def test_exp_is_correctly_rounded_f32():
    """The oracle's e^x (silu, sigmoid, softplus, decay, softmax) is the f32
    nearest to the exact value: numpy's float64 exp rounded once to f32, on
    values across the whole finite range (including the subnormal results
    and the overflow edge)."""
    from oracle import pyoracle as ora

    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-104, 89, 200000), rng.normal(0, 3, 200000), [0.0, -0.0, 1.0, -1.0, 88.72, -103.9]])
    x = x.astype(np.float32)
    got = ora.exp_f32(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
