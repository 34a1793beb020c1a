"""The chunkwise form of the gated delta rule that gdn_chunk_kernel (prefill
of sequences of >= 32 rows) computes, restated in float64 numpy and checked
against the oracle's per-token recurrence (oracle.c, qwen3_5.rs:1330-1383),
on the CPU: several chunks, a ragged last chunk, nonzero starting states,
decay near 1 and near 0. Over a chunk of m tokens from state S0, with G_t the
running sum of the log decay from the chunk start and gamma_t = exp(G_t):
  d_t = U_t - sum_{i<t} L_ti d_i,  U_t = beta_t (v_t - gamma_t S0^T k_t),
                                   L_ti = beta_t exp(G_t - G_i) (k_t . k_i)
  o_t = gamma_t S0^T q_t + sum_{i<=t} exp(G_t - G_i) (q_t . k_i) d_i
  S_m = gamma_m S0 + sum_i exp(G_m - G_i) k_i d_i^T
A wrong sign, a transposed product or a decay factor off by one token fails
this against the sequential recurrence."""
import numpy as np
import pytest

from oracle import pyoracle as ora

C = 32  # tokens per chunk, as the kernel


def softplus(x):
    return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))


def chunked_head(q, k, v, g, beta, S):
    """One value head over a sequence: q, k [n, d] (normalized, q scaled),
    v [n, dv], g (log decay) and beta [n], S [d, dv] updated in place;
    returns the raw outputs [n, dv] (before the gated norm)."""
    n = q.shape[0]
    out = np.zeros((n, v.shape[1]))
    for t0 in range(0, n, C):
        m = min(C, n - t0)
        qc, kc, vc = q[t0:t0 + m], k[t0:t0 + m], v[t0:t0 + m]
        G = np.cumsum(g[t0:t0 + m])
        gam = np.exp(G)
        bc = beta[t0:t0 + m]
        W = np.exp(G[:, None] - G[None, :])  # exp(G_t - G_i)
        L = np.tril(bc[:, None] * W * (kc @ kc.T), -1)
        B = np.tril(W * (qc @ kc.T))
        U = bc[:, None] * (vc - gam[:, None] * (kc @ S))
        d = np.zeros_like(U)
        for t in range(m):
            d[t] = U[t] - L[t, :t] @ d[:t]
        out[t0:t0 + m] = gam[:, None] * (qc @ S) + B @ d
        S[:] = gam[-1] * S + kc.T @ (np.exp(G[-1] - G)[:, None] * d)
    return out


def run_chunked(conv, a, b, z, a_log, dtb, norm, kh, vh, d, state):
    n = conv.shape[0]
    qs = conv[:, :kh * d].reshape(n, kh, d).astype(np.float64)
    ks = conv[:, kh * d:2 * kh * d].reshape(n, kh, d).astype(np.float64)
    vs = conv[:, 2 * kh * d:].reshape(n, vh, d).astype(np.float64)
    out = np.zeros((n, vh * d))
    for h in range(vh):
        kk = ks[:, h // (vh // kh)]
        qq = qs[:, h // (vh // kh)]
        kk = kk / np.sqrt((kk * kk).sum(1, keepdims=True) + 1e-6)
        qq = qq / np.sqrt((qq * qq).sum(1, keepdims=True) + 1e-6) / np.sqrt(d)
        g = -np.exp(float(a_log[h])) * softplus(a[:, h].astype(np.float64) + float(dtb[h]))
        beta = 1 / (1 + np.exp(-b[:, h].astype(np.float64)))
        S = state[h].astype(np.float64)
        o = chunked_head(qq, kk, vs[:, h], g, beta, S)
        state[h] = S
        zz = z[:, h * d:(h + 1) * d].astype(np.float64)
        o = o / np.sqrt((o * o).mean(1, keepdims=True) + 1e-6) * norm * (zz / (1 + np.exp(-zz)))
        out[:, h * d:(h + 1) * d] = o
    return out


@pytest.mark.parametrize("n,a_log_lo,a_log_hi", [(32, 0.0, 2.7), (75, 0.0, 2.7), (100, -8.0, -6.0), (40, 2.0, 3.0)])
def test_chunkwise_form_equals_recurrence(n, a_log_lo, a_log_hi):
    rng = np.random.default_rng(n)
    kh, vh, d = 2, 4, 128
    conv = rng.normal(0, 1, (n, 2 * kh * d + vh * d)).astype(np.float32)
    a = rng.normal(0, 1, (n, vh)).astype(np.float32)
    b = rng.normal(0, 1, (n, vh)).astype(np.float32)
    z = rng.normal(0, 1, (n, vh * d)).astype(np.float32)
    a_log = rng.uniform(a_log_lo, a_log_hi, vh).astype(np.float32)
    dtb = rng.normal(0, 0.1, vh).astype(np.float32)
    norm = rng.uniform(0.5, 1.5, d).astype(np.float32)
    s0 = (rng.normal(0, 1, (vh, d, d)) * 0.1).astype(np.float32)
    st_ref = s0.copy()
    ref = ora.gdn_step(conv, a, b, z, a_log, dtb, norm, kh, vh, d, d, st_ref)
    st = s0.astype(np.float64)
    got = run_chunked(conv, a, b, z, a_log, dtb, norm, kh, vh, d, st)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 1e-4 * scale
    assert np.abs(st - st_ref).max() <= 1e-4 * np.abs(st_ref).max()
