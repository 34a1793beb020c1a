"""Q8_0 / Q5_0 matrices (GGML 32-weight blocks, the types a Q4_K_M GGUF holds
for rows that are not whole 256-weight super-blocks) through the C ABI.

Bars: dequantized weights bit-exact to the oracle; GEMV (store, residual,
fused SwiGLU) within 1e-3 of an fp64 dot over the oracle-dequantized
weights; batched rows bitwise equal to one-row calls; a Qwen2 model whose
320-wide rows are Q5_0 / Q8_0 and whose 512-wide rows are Q4_K / Q6_K,
loaded from a GGUF file, matches the oracle holding the same blocks.
"""
import numpy as np
import pytest

from checkpoints import (GGML_Q5_0, GGML_Q8_0, K_EMBED, K_GATE, K_K, K_O, K_Q, K_UP, K_V, ORACLE_FMT,
                         gguf_tensors_from_oracle, qwen2_meta, random_blocks, write_gguf)
from oracle import pyoracle as ora
from test_gpu_model import LOGIT_TOL, oracle2, rel, small2

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
TYPES = {"q8_0": (GGML_Q8_0, 3), "q5_0": (GGML_Q5_0, 4)}


def rel_err(y, ref):
    return float(np.abs(y.astype(np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def make(dev, name, n_out, n_in, seed):
    from pagoda_amd import Matrix

    gt, fmt = TYPES[name]
    blk = random_blocks(np.random.default_rng(seed), gt, n_out, n_in)
    deq = (ora.q8_0_dequant if name == "q8_0" else ora.q5_0_dequant)(blk, n_out, n_in)
    return Matrix.upload_kq(dev, fmt, blk, n_out, n_in), deq


@pytest.mark.parametrize("name", ["q8_0", "q5_0"])
@pytest.mark.parametrize("shape", [(5, 32), (37, 896), (64, 4864)])
def test_block_dequant_bit_exact(dev, name, shape):
    m, deq = make(dev, name, *shape, seed=shape[0])
    try:
        assert m.fmt == TYPES[name][1]
        np.testing.assert_array_equal(m.dequant().view(np.uint32), deq.view(np.uint32))
        # a row window (the embedding lookup path)
        np.testing.assert_array_equal(m.dequant(2, 3).view(np.uint32), deq[2:5].view(np.uint32))
    finally:
        m.free()


@pytest.mark.parametrize("name", ["q8_0", "q5_0"])
@pytest.mark.parametrize("x_f16", [False, True])
def test_block_gemv(dev, name, x_f16):
    n_out, n_in = 200, 896
    m, deq = make(dev, name, n_out, n_in, seed=7)
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (40, n_in)).astype(np.float16 if x_f16 else np.float32)
    res = rng.normal(0, 1, (40, n_out)).astype(np.float32)
    xd, rd, yd = dev.upload(x), dev.upload(res), dev.alloc(40 * n_out * 4)
    try:
        outs = {}
        for rows in (1, 3, 8, 17, 40):
            m.gemv_dev(xd, n_in, rows, yd, n_out, x_f16=x_f16)
            outs[rows] = dev.download(yd, (rows, n_out), np.float32)
            ref = x[:rows].astype(np.float64) @ deq.astype(np.float64).T
            assert rel_err(outs[rows], ref) < GEMV_TOL, rows
        for rows in (3, 8, 17, 40):
            np.testing.assert_array_equal(outs[rows][0].view(np.uint32), outs[1][0].view(np.uint32))
        np.testing.assert_array_equal(outs[40][:17].view(np.uint32), outs[17].view(np.uint32))
        # residual epilogue: y = res + W x
        m.gemv_dev(xd, n_in, 17, yd, n_out, x_f16=x_f16, res_ptr=rd, ldres=n_out)
        got = dev.download(yd, (17, n_out), np.float32)
        ref = res[:17].astype(np.float64) + x[:17].astype(np.float64) @ deq.astype(np.float64).T
        assert rel_err(got, ref) < GEMV_TOL
    finally:
        for p in (xd, rd, yd):
            dev.free(p)
        m.free()


@pytest.mark.parametrize("name", ["q8_0", "q5_0"])
def test_block_swiglu(dev, name):
    from pagoda_amd import Matrix

    n_out, n_in = 160, 320
    g, gd = make(dev, name, n_out, n_in, seed=11)
    u, ud = make(dev, name, n_out, n_in, seed=12)
    x = np.random.default_rng(4).normal(0, 1, (9, n_in)).astype(np.float32)
    xd, md = dev.upload(x), dev.alloc(9 * n_out * 4)
    try:
        Matrix.gemv_swiglu_dev(g, u, xd, n_in, 9, md, n_out)
        got = dev.download(md, (9, n_out), np.float32)
        a = x.astype(np.float64) @ gd.astype(np.float64).T
        b = x.astype(np.float64) @ ud.astype(np.float64).T
        assert rel_err(got, a / (1.0 + np.exp(-a)) * b) < GEMV_TOL
    finally:
        dev.free(xd)
        dev.free(md)
        g.free()
        u.free()


def test_gguf_fallback_block_types_match_oracle(dev, tmp_path):
    """The Q4_K_M layout of a model whose hidden size is not a multiple of
    256 (Qwen2.5-0.5B: 896): the 320-wide rows (embedding, q/k/v/o, gate/up)
    are Q5_0 / Q8_0, the 512-wide ffn_down rows keep Q4_K / Q6_K. Layer 0's q
    and k share a type (one stacked matrix), layer 1's do not."""
    from pagoda_amd.engine import Model

    cfg = small2(hidden=320, heads=5, kv_heads=1, head_dim=64, intermediate=512, n_layers=2)
    oracle = oracle2(cfg, 9)
    rng = np.random.default_rng(10)
    H, kvw, qw = cfg.hidden, cfg.kv_heads * cfg.head_dim, cfg.heads * cfg.head_dim
    types = {(-1, K_EMBED): GGML_Q8_0}
    for i in range(cfg.n_layers):
        # layer 0: q and k in one type (one stacked matrix); layer 1: different types (two matrices)
        types.update({(i, K_Q): GGML_Q5_0, (i, K_K): GGML_Q5_0 if i == 0 else GGML_Q8_0, (i, K_V): GGML_Q8_0,
                      (i, K_O): GGML_Q5_0,
                      (i, K_GATE): GGML_Q5_0, (i, K_UP): GGML_Q5_0})
    shapes = {K_EMBED: (cfg.vocab, H), K_Q: (qw, H), K_K: (kvw, H), K_V: (kvw, H), K_O: (H, qw),
              K_GATE: (cfg.intermediate, H), K_UP: (cfg.intermediate, H)}
    for (layer, kind), gt in types.items():
        oracle.set_matrix(layer, kind, ORACLE_FMT[gt], random_blocks(rng, gt, *shapes[kind]))
    p = tmp_path / "fallback.gguf"
    write_gguf(p, qwen2_meta(cfg), gguf_tensors_from_oracle(cfg, oracle, types=types))
    model = Model.load_gguf(dev, p, kv_blocks=cfg.kv_blocks)
    s = model.new_session()
    try:
        c = oracle.new_cache()
        prompt = np.random.default_rng(11).integers(0, cfg.vocab, 9)
        got, ref = s.forward(prompt), oracle.forward(prompt, c)
        for step in range(8):
            assert rel(got, ref) < LOGIT_TOL, f"step {step}: {rel(got, ref)}"
            tok = int(np.argmax(ref))
            assert int(np.argmax(got)) == tok, f"greedy token diverged at step {step}"
            got, ref = s.forward([tok]), oracle.forward([tok], c)
    finally:
        s.free()
        model.free()
