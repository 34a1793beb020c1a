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


# ------------------------------------------------- engine-addressable KV pages
def _bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


@pytest.mark.parametrize("k", [16, 21, 37])
def test_session_from_pages_equals_fork_prefix(dev, k):
    """The radix-cache flow of pagoda/src/radix_cache.rs over device pages: a
    finished request's pages are retained by the engine (inc_ref), its session
    is freed, and a later request whose prompt shares the first k tokens is
    built from those page ids without a copy. It decodes bit for bit like a
    prefix graft of the original, the original's KV is never disturbed by the
    new session's writes (copy-on-write of the shared partial page), and
    every page goes back to the pool once every holder let go."""
    from pagoda_amd.engine import Model

    cfg = small2(kv_blocks=64)
    model = Model.synth(dev, cfg, 5)
    try:
        pool = model.kv_pool()
        assert pool == {"pages": 64, "page_tokens": 16, "free": 64}
        toks = np.random.default_rng(9).integers(0, cfg.vocab, 40)
        s = model.new_session()
        s.forward(toks)
        pages = s.pages()
        assert pages.size == 3 and len(set(pages.tolist())) == 3
        assert all(model.page_refcount(p) == 1 for p in pages)
        g = s.fork_prefix(k)
        before = s.export_kv()
        # engine side: the radix cache takes its references on the pages that
        # hold the first k positions (ceil(k / 16))
        held = pages[: (k + 15) // 16]
        model.page_retain(held)
        assert all(model.page_refcount(p) == 3 for p in held)  # s, g, engine
        t = model.session_from_pages(held, k)
        assert t.context_len() == k
        np.testing.assert_array_equal(t.pages(), held)
        cont = [11, 12, 13, 14, 15, 16, 17, 18, 19]
        np.testing.assert_array_equal(_bits(t.forward(cont)), _bits(g.forward(cont)))
        for tok in (3, 7, 1):
            np.testing.assert_array_equal(_bits(t.forward([tok])), _bits(g.forward([tok])))
        assert s.export_kv() == before
        # the engine's pages still hold the original KV: a second session
        # built from them later decodes like the first one did
        u = model.session_from_pages(held, k)
        t2 = s.fork_prefix(k)
        np.testing.assert_array_equal(_bits(u.forward(cont)), _bits(t2.forward(cont)))
        for x in (s, g, t, u, t2):
            x.free()
        assert all(model.page_refcount(p) == 1 for p in held)  # the engine's own
        model.page_release(held)
        assert all(model.page_refcount(p) == 0 for p in pages)
        assert model.kv_pool()["free"] == 64
    finally:
        model.free()


def test_session_from_pages_errors(dev):
    from pagoda_amd import PagodaError
    from pagoda_amd.engine import Model

    model = Model.synth(dev, small2(kv_blocks=32), 5)
    try:
        s = model.new_session()
        s.forward(np.arange(20))
        p = s.pages()
        free_page = next(i for i in range(32) if model.page_refcount(i) == 0)
        bad = [
            (p, 33),                      # 33 positions need 3 pages
            (p[:1], 20),                  # 20 positions need 2
            ([p[0], p[0]], 20),           # a page listed twice
            ([p[0], free_page], 20),      # a free page
            ([p[0], 99], 20),             # outside the pool
        ]
        for ids, n in bad:
            with pytest.raises(PagodaError):
                model.session_from_pages(ids, n)
        with pytest.raises(PagodaError):
            model.page_retain([free_page])
        with pytest.raises(PagodaError):
            model.page_release([p[0], p[0]])  # held once
        assert model.page_refcount(p[0]) == 1
        e = model.session_from_pages([], 0)
        assert e.context_len() == 0 and e.pages().size == 0
        e.free()
        s.free()
    finally:
        model.free()
    hy = Model.synth(dev, small35(n_layers=4), 11)
    try:
        h = hy.new_session()
        h.forward([1, 2, 3])
        hp = h.pages()
        with pytest.raises(PagodaError) as ei:
            hy.session_from_pages(hp, 3)
        assert ei.value.code == -5
        h.free()
    finally:
        hy.free()


def test_pool_exhaustion_leaves_sessions_usable(dev):
    """A step that cannot get KV pages fails with PGD_ERR_ALLOC before any
    state is written: no session advances or is poisoned, and both continue
    exactly like twins that never saw the failed step (atomic batched step,
    pagoda-hf/src/llama.rs:750-778)."""
    from pagoda_amd import PagodaError
    from pagoda_amd.engine import Model

    model = Model.synth(dev, small2(kv_blocks=6), 5)
    try:
        rng = np.random.default_rng(12)
        a_t, b_t = rng.integers(0, 1024, 30), rng.integers(0, 1024, 40)
        a, b = model.new_session(), model.new_session()
        a.forward(a_t)
        b.forward(b_t)  # 2 + 3 pages of 6
        ta, tb = a.fork(), b.fork()  # share the pages: no new ones
        with pytest.raises(PagodaError) as ei:
            model.step_ragged([a, b], [rng.integers(0, 1024, 20), [5]])  # a needs 2 more, 1 free
        assert ei.value.code == -6
        assert (a.context_len(), b.context_len()) == (30, 40)
        # the failed step took no pages for good either: a twin-for-twin
        # continuation needs and finds them
        for x, y in ((a, ta), (b, tb)):
            np.testing.assert_array_equal(_bits(x.forward([9])), _bits(y.forward([9])))
            x.free()
            y.free()
        assert model.kv_pool()["free"] == 6
    finally:
        model.free()
