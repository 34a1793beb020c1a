"""Session surface beyond the forward: the Qwen2 SessionKv PD payload
(pagoda-hf/src/llama.rs:215-345) against the oracle in both directions, the
prefix graft (cache_prefix, pagoda-hf/src/lib.rs:219-226, 603-616), and the
engine's per-request fault on non-finite logits (pagoda/src/engine.rs:
1270-1280)."""
import numpy as np
import pytest

import sessionkv
from oracle import pyoracle as ora
from test_gpu_model import LOGIT_TOL, oracle2, rel, small2, small35

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def q2(dev):
    from pagoda_amd.engine import Model

    cfg = small2()
    m = Model.synth(dev, cfg, 5)
    yield m, oracle2(cfg, 5)


def _close(x, y, tol=1e-3):
    x, y = x.astype(np.float64), y.astype(np.float64)
    scale = max(np.abs(y).max(), 1e-30)
    assert np.abs(x - y).max() <= tol * scale
    assert np.all(np.abs(x - y) <= tol * np.abs(y) + 1e-4 * scale)


def test_qwen2_export_matches_oracle_payload(q2):
    model, oracle = q2
    prompt = np.random.default_rng(2).integers(0, model.cfg.vocab, 21)
    s = model.new_session()
    logits = s.forward(prompt)
    g = s.export_kv()
    oc = oracle.new_cache()
    ref_logits = oracle.forward(prompt, oc)
    r = oc.export_bytes(ref_logits)
    assert len(g) == len(r)
    G, R = sessionkv.parse(g), sessionkv.parse(r)
    assert (G["version"], G["len"], len(G["layers"]), G["trailing"]) == (2, 21, model.cfg.n_layers, 0)
    assert (R["version"], R["len"], len(R["layers"])) == (G["version"], G["len"], len(G["layers"]))
    np.testing.assert_array_equal(G["logits"], logits)  # the session's own last logits, f32-exact
    _close(G["logits"], R["logits"])
    for a, b in zip(G["layers"], R["layers"]):
        assert (a["kv_heads"], a["head_dim"], a["dtype"]) == (b["kv_heads"], b["head_dim"], b["dtype"])
        _close(a["k"], b["k"])
        _close(a["v"], b["v"])
    s.free()


def test_qwen2_import_oracle_payload_continues_like_oracle(q2):
    model, oracle = q2
    prompt = np.random.default_rng(3).integers(0, model.cfg.vocab, 19)
    oc = oracle.new_cache()
    ref = oracle.forward(prompt, oc)
    t = model.import_session(oc.export_bytes(ref))
    assert t.context_len() == 19
    # an empty feed replays the payload's logits (pagoda-hf/src/lib.rs:644-667)
    np.testing.assert_array_equal(t.forward([]), ref)
    tok = ora.argmax_first(ref)
    for k in range(4):
        g = t.forward([tok])
        r = oracle.forward([tok], oc)
        assert rel(g, r) < LOGIT_TOL, k
        assert ora.argmax_first(g) == ora.argmax_first(r), k
        tok = ora.argmax_first(r)
    t.free()


def test_qwen2_gpu_payload_continues_in_oracle(q2):
    model, oracle = q2
    prompt = np.random.default_rng(4).integers(0, model.cfg.vocab, 17)
    s = model.new_session()
    s.forward(prompt)
    blob = s.export_kv()
    u = model.import_session(blob)
    assert u.export_kv() == blob  # bitwise round trip through the device
    oc, lg = ora.Qwen2Cache.import_bytes(oracle, blob)
    assert len(oc) == 17 and lg is not None
    tok = 3
    for k in range(4):
        g = u.forward([tok])
        r = oracle.forward([tok], oc)
        assert rel(g, r) < LOGIT_TOL, k
        assert ora.argmax_first(g) == ora.argmax_first(r), k
        tok = ora.argmax_first(r)
    s.free()
    u.free()


def test_qwen2_f16_wire(q2):
    from pagoda_amd.engine import set_kv_wire_f16

    model, oracle = q2
    prompt = np.random.default_rng(5).integers(0, model.cfg.vocab, 9)
    s = model.new_session()
    s.forward(prompt)
    b32 = s.export_kv()
    set_kv_wire_f16(True)
    try:
        b16 = s.export_kv()
    finally:
        set_kv_wire_f16(False)
    c = model.cfg
    assert len(b16) == len(b32) - c.n_layers * c.kv_heads * 9 * c.head_dim * 2 * 2
    p32, p16 = sessionkv.parse(b32), sessionkv.parse(b16)
    np.testing.assert_array_equal(p16["logits"], p32["logits"])
    for a, b in zip(p32["layers"], p16["layers"]):
        assert b["dtype"] == 1
        np.testing.assert_array_equal(b["k"].view(np.uint16), a["k"].astype(np.float16).view(np.uint16))
        np.testing.assert_array_equal(b["v"].view(np.uint16), a["v"].astype(np.float16).view(np.uint16))
    # the f16 payload imports and equals the oracle fed the same f16 values
    t = model.import_session(b16)
    oc, _ = ora.Qwen2Cache.import_bytes(oracle, b16)
    g, r = t.forward([7]), oracle.forward([7], oc)
    assert rel(g, r) < LOGIT_TOL
    s.free()
    t.free()


def test_qwen2_import_rejects_malformed(q2):
    from pagoda_amd import PagodaError

    model, _ = q2
    s = model.new_session()
    s.forward([1, 2, 3])
    blob = s.export_kv()
    c = model.cfg
    wrong_heads = sessionkv.write(3, [(np.zeros((1, 3, c.head_dim)),) * 2] * c.n_layers)
    for bad in (blob[:12], b"garbage", b"\0" + blob[1:], blob[:4] + b"\x03" + blob[5:], blob[:-1], wrong_heads):
        with pytest.raises(PagodaError):
            model.import_session(bad)
    s.free()


@pytest.mark.parametrize("n", [0, 5, 16, 17, 40])
def test_fork_prefix_equals_fresh_prefix(q2, n):
    """A prefix graft is bit-identical to a session fed only the prefix
    (causality, llama.rs:81-87), and appends to it leave the original intact."""
    model, _ = q2
    toks = np.random.default_rng(6).integers(0, model.cfg.vocab, 40)
    full = model.new_session()
    full.forward(toks)
    before = full.export_kv()
    p = full.fork_prefix(n)
    assert p.context_len() == n
    fresh = model.new_session()
    if n:
        fresh.forward(toks[:n])
    cont = [11, 12, 13, 14, 15, 16, 17, 18, 19, 20]
    np.testing.assert_array_equal(p.forward(cont).view(np.uint32), fresh.forward(cont).view(np.uint32))
    np.testing.assert_array_equal(p.forward([3]).view(np.uint32), fresh.forward([3]).view(np.uint32))
    assert full.export_kv() == before
    for x in (full, p, fresh):
        x.free()


def test_fork_prefix_errors(q2, dev):
    from pagoda_amd import PagodaError
    from pagoda_amd.engine import HipEngine, Model

    model, _ = q2
    s = model.new_session()
    s.forward([1, 2, 3])
    with pytest.raises(PagodaError):
        s.fork_prefix(4)
    with pytest.raises(PagodaError):
        s.fork_prefix(-1)
    s.free()
    hy = Model.synth(dev, small35(n_layers=4), 11)
    h = hy.new_session()
    h.forward([1, 2, 3])
    with pytest.raises(PagodaError, match="prefix"):
        h.fork_prefix(2)
    assert HipEngine(hy).graft_session(h, 2) is None
    h.free()
    hy.free()


# ------------------------------------------------------------ non-finite rows
def _poisoned_mlx(dev, tmp_path, edit):
    from checkpoints import mlx_tensors_from_oracle, mlx_text_config, write_mlx_config, write_safetensors_shards
    from pagoda_amd.engine import Model
    from test_gpu_model import oracle35

    cfg = small35(n_layers=4)
    t = mlx_tensors_from_oracle(cfg, oracle35(cfg, 11))
    edit(t)
    d = tmp_path / "mlx"
    write_mlx_config(d, mlx_text_config(cfg, max_pos=cfg.max_pos))
    write_safetensors_shards(d, t, nshards=2)
    return Model.load_mlx(dev, d, kv_blocks=cfg.kv_blocks), Model.synth(dev, cfg, 11)


def test_nan_embedding_row_faults_only_its_request(dev, tmp_path):
    bad_tok = 77

    def edit(t):
        t["language_model.model.embed_tokens.scales"][1][bad_tok] = 0x7FC0  # bf16 NaN

    model, clean = _poisoned_mlx(dev, tmp_path, edit)
    try:
        feeds = [[5, 9, 2], [bad_tok], [31, 8]]
        ss = [model.new_session() for _ in feeds]
        ids, logits = model.step_ragged(ss, feeds, want_logits=True)
        cs = [clean.new_session() for _ in feeds]
        cfeeds = [feeds[0], [78], feeds[2]]
        cids, clog = clean.step_ragged(cs, cfeeds, want_logits=True)
        assert ids[1] == 0xFFFFFFFF and not np.isfinite(logits[1]).all()
        for i in (0, 2):
            assert ids[i] == cids[i] != 0xFFFFFFFF
            np.testing.assert_array_equal(logits[i].view(np.uint32), clog[i].view(np.uint32))
        for s in ss + cs:
            s.free()
    finally:
        model.free()
        clean.free()


def test_one_nonfinite_logit_faults_the_row(dev, tmp_path):
    """A single non-finite logit (lm_head row 7 with an infinite bias) faults
    every request: the rule is any non-finite value, not all."""
    def edit(t):
        t["language_model.lm_head.biases"][1][7, :] = 0x7F80  # bf16 +inf
        t["language_model.lm_head.scales"][1][7, :] = 0

    model, clean = _poisoned_mlx(dev, tmp_path, edit)
    try:
        feeds = [[5, 9, 2], [4], [31, 8]]
        ss = [model.new_session() for _ in feeds]
        ids, logits = model.step_ragged(ss, feeds, want_logits=True)
        for i in range(3):
            assert not np.isfinite(logits[i][7])
            assert np.isfinite(np.delete(logits[i], 7)).all()
            assert ids[i] == 0xFFFFFFFF
        g, _ = ss[0].forward_greedy(3)
        assert g == 0xFFFFFFFF
        for s in ss:
            s.free()
    finally:
        model.free()
        clean.free()
