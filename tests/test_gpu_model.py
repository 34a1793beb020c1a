"""End-to-end decode parity of the HIP backend against the CPU oracle on
identical seeded weights (small configs here; the full configs are in
test_gpu_configs.py)."""
import numpy as np
import pytest

from oracle import pyoracle as ora

import cachev1

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3  # max |diff| / max |ref| per logits vector


def rel(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def small35(**kw):
    from pagoda_amd.engine import ModelConfig

    c = dict(arch=0, n_layers=8, hidden=256, intermediate=512, vocab=1024, heads=4, kv_heads=2, head_dim=128,
             rotary_dim=32, rope_theta=1e7, eps=1e-6, k_heads=2, v_heads=4, k_dim=128, v_dim=128, conv_kernel=4,
             full_every=4, max_pos=512, kv_block=16, kv_blocks=256)
    c.update(kw)
    return ModelConfig(**c)


def small2(**kw):
    from pagoda_amd.engine import ARCH_QWEN2, ModelConfig

    c = dict(arch=ARCH_QWEN2, n_layers=3, hidden=256, intermediate=640, vocab=1024, heads=4, kv_heads=2, head_dim=64,
             rotary_dim=64, rope_theta=1e6, eps=1e-6, k_heads=0, v_heads=0, k_dim=0, v_dim=0, conv_kernel=0,
             full_every=1, max_pos=512, kv_block=16, kv_blocks=256)
    c.update(kw)
    return ModelConfig(**c)


def oracle35(cfg, seed):
    return ora.Qwen35(ora.Qwen35Config(
        n_layers=cfg.n_layers, hidden=cfg.hidden, intermediate=cfg.intermediate, vocab=cfg.vocab, heads=cfg.heads,
        kv_heads=cfg.kv_heads, head_dim=cfg.head_dim, rotary_dim=cfg.rotary_dim, rope_theta=cfg.rope_theta,
        k_heads=cfg.k_heads, v_heads=cfg.v_heads, k_dim=cfg.k_dim, v_dim=cfg.v_dim, conv_kernel=cfg.conv_kernel,
        full_every=cfg.full_every), seed)


def oracle2(cfg, seed):
    return ora.Qwen2(ora.Qwen2Config(
        n_layers=cfg.n_layers, hidden=cfg.hidden, intermediate=cfg.intermediate, vocab=cfg.vocab, heads=cfg.heads,
        kv_heads=cfg.kv_heads, head_dim=cfg.head_dim, max_pos=cfg.max_pos, rope_theta=cfg.rope_theta, eps=cfg.eps),
        seed)


@pytest.fixture(scope="module")
def m35(dev):
    from pagoda_amd.engine import Model

    cfg = small35()
    m = Model.synth(dev, cfg, 11)
    yield m, oracle35(cfg, 11)


@pytest.fixture(scope="module")
def m2(dev):
    from pagoda_amd.engine import Model

    cfg = small2()
    m = Model.synth(dev, cfg, 5)
    yield m, oracle2(cfg, 5)


@pytest.mark.parametrize("which", ["m35", "m2"])
def test_prefill_then_greedy_decode_matches_oracle(which, request):
    model, oracle = request.getfixturevalue(which)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, model.cfg.vocab, 11)
    s = model.new_session()
    oc = oracle.new_cache()
    got = s.forward(prompt)
    ref = oracle.forward(prompt, oc)
    assert rel(got, ref) < LOGIT_TOL
    tok = int(np.argmax(ref))
    for step in range(16):
        assert int(np.argmax(got)) == int(np.argmax(ref)), f"greedy token diverged at step {step}"
        got = s.forward([tok])
        ref = oracle.forward([tok], oc)
        assert rel(got, ref) < LOGIT_TOL, f"step {step}: {rel(got, ref)}"
        tok = int(np.argmax(ref))
    assert s.context_len() == 11 + 16
    # empty feed replays the cached logits (pagoda/src/model.rs:153-157)
    np.testing.assert_array_equal(s.forward([]), got)


@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_qwen2_cpu_arithmetic_bitwise_every_head_dim(dev, head_dim):
    """The Qwen2 default arithmetic (candle's quantized matmul and the CPU
    path's attention order, qwen2_gguf.rs:252-289) at every head size the
    exact-order attention kernel takes: prompt and 12 greedy steps bit-equal
    to the oracle's restatement on the same weights."""
    from pagoda_amd.engine import ARITH_CPU_Q8, Model, argmax_first

    cfg = small2(head_dim=head_dim, rotary_dim=head_dim, n_layers=2)
    print(f"qwen2 cpu_q8 head_dim {head_dim}", flush=True)
    m = Model.synth(dev, cfg, 21)
    m.set_kquant_arith(ARITH_CPU_Q8)
    o = oracle2(cfg, 21)
    rng = np.random.default_rng(head_dim)
    prompt = rng.integers(0, cfg.vocab, 37)
    s = m.new_session()
    oc = o.new_cache()
    got = s.forward(prompt)
    ref = o.forward(prompt, oc)
    for step in range(12):
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32), err_msg=f"step {step}")
        t = argmax_first(got)
        assert t == ora.argmax_first(ref)
        got = s.forward([t])
        ref = o.forward([t], oc)
    s.free()
    m.free()


@pytest.mark.parametrize("which", ["m35", "m2"])
def test_ragged_batch_bitwise_equals_serial(which, request):
    """Batched step == per-session forwards (pagoda/tests/batch_tests.rs:217-242).
    Every kernel computes rows independently. A row's logits are bitwise equal
    whenever the GEMV launches holding it have the same size class (1..4 or
    5..32 rows: the fused SwiGLU and the >= 2048-tile lm_head switch kernels
    between them), else within 1e-5 with the same greedy id; a permuted batch
    is bitwise equal to the original."""
    model, _ = request.getfixturevalue(which)
    rng = np.random.default_rng(4)
    prompts = [rng.integers(0, model.cfg.vocab, n) for n in (5, 9, 1, 17)]
    serial = [model.new_session() for _ in prompts]
    batched = [model.new_session() for _ in prompts]
    permuted = [model.new_session() for _ in prompts]
    order = [2, 0, 3, 1]

    def check(bl, ser, feeds):
        for i in range(len(feeds)):
            same_class = (len(feeds[i]) <= 4) == (sum(len(f) for f in feeds) <= 4)
            if same_class:
                np.testing.assert_array_equal(bl[i].view(np.uint32), ser[i].view(np.uint32))
            else:
                assert rel(bl[i], ser[i]) < 1e-5
                assert int(np.argmax(bl[i])) == int(np.argmax(ser[i]))

    ser_logits = [s.forward(p) for s, p in zip(serial, prompts)]
    _, bl = model.step_ragged(batched, prompts, want_logits=True)
    check(bl, ser_logits, prompts)
    _, pl = model.step_ragged([permuted[i] for i in order], [prompts[i] for i in order], want_logits=True)
    for k, i in enumerate(order):
        np.testing.assert_array_equal(pl[k].view(np.uint32), bl[i].view(np.uint32))
    # mixed decode rows and 4-token chunks in one step
    feeds = [[int(np.argmax(ser_logits[0]))], rng.integers(0, model.cfg.vocab, 4), [7], rng.integers(0, 100, 3)]
    ser = [s.forward(f) for s, f in zip(serial, feeds)]
    _, bl = model.step_ragged(batched, feeds, want_logits=True)
    check(bl, ser, feeds)
    assert [s.context_len() for s in batched] == [s.context_len() for s in serial]


def test_small_decode_batch_bitwise_equals_serial(m35):
    """Steps of 2..4 decode rows, one per sequence: the projection GEMV runs
    each row's causal conv in its epilogue on that sequence's state. Three
    sequences stepped together equal each stepped alone (one-row launches),
    bitwise, over two steps."""
    model, _ = m35
    rng = np.random.default_rng(13)
    prompts = [rng.integers(0, model.cfg.vocab, n) for n in (3, 6, 2)]
    batched = [model.new_session() for _ in prompts]
    serial = []
    try:
        for s, p in zip(batched, prompts):
            s.forward(p)
        serial = [s.fork() for s in batched]
        toks = [int(t) for t in rng.integers(0, model.cfg.vocab, 3)]
        for _ in range(2):
            _, bl = model.step_ragged(batched, [[t] for t in toks], want_logits=True)
            sl = [s.forward([t]) for s, t in zip(serial, toks)]
            for i in range(3):
                np.testing.assert_array_equal(bl[i].view(np.uint32), sl[i].view(np.uint32))
            toks = [int(np.argmax(x)) for x in sl]
    finally:
        for x in batched + serial:
            x.free()


def test_verify_equals_serial_greedy(m35):
    """forward_verify(4) == 4 serial greedy steps (pagoda-hf/examples/qwen3_8.rs:219-247)."""
    model, _ = m35
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, model.cfg.vocab, 6)
    a = model.new_session()
    a.forward(prompt[:-1])
    b = a.fork()
    inp = int(prompt[-1])
    produced = []
    for _ in range(4):
        t, v = a.forward_greedy(inp)
        produced.append((t, v))
        inp = t
    inputs = [int(prompt[-1])] + [t for t, _ in produced[:3]]
    got = b.forward_verify(inputs)
    assert [t for t, _ in got] == [t for t, _ in produced]
    for (_, v1), (_, v2) in zip(got, produced):
        assert v1 == v2  # same per-row kernels: bitwise
    assert a.context_len() == b.context_len()


def test_fork_continues_independently(m35):
    model, oracle = m35
    rng = np.random.default_rng(6)
    prompt = rng.integers(0, model.cfg.vocab, 21)  # crosses a 16-token page
    s = model.new_session()
    s.forward(prompt)
    f = s.fork()
    a1 = s.forward([3, 4])
    b1 = f.forward([3, 4])
    np.testing.assert_array_equal(a1, b1)
    a2 = s.forward([9])
    b2 = f.forward([10])  # diverge: the shared tail page is copied on write
    a3 = s.forward([5])
    oc = oracle.new_cache()
    oracle.forward(prompt, oc)
    oracle.forward([3, 4], oc)
    ref_b2 = oracle.forward([10], oc.clone())
    ref_a2 = oracle.forward([9], oc)
    ref_a3 = oracle.forward([5], oc)
    assert rel(a2, ref_a2) < LOGIT_TOL and rel(b2, ref_b2) < LOGIT_TOL and rel(a3, ref_a3) < LOGIT_TOL
    f.free()


def _assert_cache_bytes_close(g: bytes, r: bytes, tol: float = 1e-3):
    """Tags, counts and integers identical; every float vector within tol of
    its reference, max-normalized and elementwise (|d| <= tol*|ref| + atol
    with atol = 1e-4 * max|ref| of that vector)."""
    G, R = cachev1.parse(g), cachev1.parse(r)
    assert G["len"] == R["len"] and len(G["layers"]) == len(R["layers"])
    for i, (a, b) in enumerate(zip(G["layers"], R["layers"])):
        assert a["tag"] == b["tag"], i
        keys = ("conv", "state") if a["tag"] == 1 else ("k", "v")
        if a["tag"] == 2:
            assert (a["kv_len"], a["kv_heads"], a["head_dim"]) == (b["kv_len"], b["kv_heads"], b["head_dim"]), i
        for key in keys:
            x, y = a[key].astype(np.float64), b[key].astype(np.float64)
            assert x.size == y.size, (i, key)
            scale = max(np.abs(y).max(), 1e-30) if y.size else 1.0
            assert np.abs(x - y).max(initial=0) <= tol * scale, (i, key)
            assert np.all(np.abs(x - y) <= tol * np.abs(y) + 1e-4 * scale), (i, key)


def test_export_import_round_trip(m35):
    """Cache bytes v1 (pagoda-hf/src/qwen3_5.rs:177-256). The GPU export and
    the oracle's to_bytes of the same prompt have identical tags, counts and
    shapes and floats within 1e-3; bytes the ORACLE wrote import into the GPU
    and decode 4 greedy steps like the oracle; bytes the GPU wrote import
    into the oracle and decode like the GPU session. So a layout shared by
    export and import but different from the reference's fails."""
    model, oracle = m35
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, model.cfg.vocab, 19)
    s = model.new_session()
    s.forward(prompt)
    blob = s.export_kv()
    oc = oracle.new_cache()
    ref_logits = oracle.forward(prompt, oc)
    ref = oc.to_bytes()
    assert len(blob) == len(ref)
    _assert_cache_bytes_close(blob, ref)
    # the GPU's own bytes round-trip bitwise
    t = model.import_session(blob)
    assert t.context_len() == 19
    assert t.export_kv() == blob
    np.testing.assert_array_equal(t.forward([1]), s.forward([1]))
    # oracle bytes -> GPU, 4 greedy steps against the oracle continuing
    u = model.import_session(ref)
    assert u.context_len() == 19
    tok = ora.argmax_first(ref_logits)
    oc2 = oc.clone()
    for k in range(4):
        g = u.forward([tok])
        r = oracle.forward([tok], oc2)
        assert rel(g, r) < LOGIT_TOL, k
        assert ora.argmax_first(g) == ora.argmax_first(r), k
        tok = ora.argmax_first(r)
    # GPU bytes -> oracle, 4 greedy steps against the GPU session continuing
    v = model.import_session(blob)
    od = ora.Qwen35Cache.from_bytes(blob, oracle)
    tok = 5
    for k in range(4):
        g = v.forward([tok])
        r = oracle.forward([tok], od)
        assert rel(g, r) < LOGIT_TOL, k
        assert ora.argmax_first(g) == ora.argmax_first(r), k
        tok = ora.argmax_first(r)
    for x in (s, t, u, v):
        x.free()


def test_import_rejects_malformed_bytes(m35):
    from pagoda_amd import PagodaError

    model, oracle = m35
    s = model.new_session()
    s.forward([1, 2, 3])
    blob = s.export_kv()
    for bad in (b"\x02" + blob[1:], blob + b"\x00", blob[:-4], blob[:16] + b"\x07" + blob[17:]):
        with pytest.raises(PagodaError):
            model.import_session(bad)
    s.free()


def test_argument_errors_are_atomic(m35):
    from pagoda_amd import PagodaError

    model, _ = m35
    s = model.new_session()
    s.forward([1, 2, 3])
    t = model.new_session()
    with pytest.raises(PagodaError):
        model.step_ragged([s, t], [[1], [model.cfg.vocab + 5]])  # bad token in one row
    assert s.context_len() == 3 and t.context_len() == 0
    with pytest.raises(PagodaError):
        model.step_ragged([s, s], [[1], [2]])  # duplicate session
    assert s.context_len() == 3
    with pytest.raises(PagodaError):
        s.forward_verify([1, 2, 3, 4, 5])


@pytest.mark.parametrize("which", ["m35", "m2"])
def test_shared_trunk_mixed_decode_and_verify(which, request):
    """Config-5 pattern at small size: requests fork one prefilled trunk
    (KV pages shared copy-on-write), prefill distinct suffixes in one ragged
    step, then decode; a second pass from the same post-suffix states packs
    1-token decode rows with 4-token known-token verify chunks into one ragged
    batch. Every verified id equals the decoded stream, and one request's
    stream equals the oracle's greedy stream on the same tokens."""
    model, oracle = request.getfixturevalue(which)
    rng = np.random.default_rng(21)
    trunk = rng.integers(0, model.cfg.vocab, 40)
    nreq, gen = 6, 9
    root = model.new_session()
    root.forward(trunk)
    reqs = [root.fork() for _ in range(nreq)]
    suffixes = [rng.integers(0, model.cfg.vocab, 3 + i) for i in range(nreq)]
    first, _ = model.step_ragged(reqs, suffixes)
    snap = [r.fork() for r in reqs]
    streams = [[int(t)] for t in first]
    for _ in range(gen - 1):
        ids, _ = model.step_ragged(reqs, [[s[-1]] for s in streams])
        for s, t in zip(streams, ids):
            s.append(int(t))
    pos = [1] * nreq
    while any(p < gen for p in pos):
        sess, feeds, owners = [], [], []
        for i in range(nreq):
            if pos[i] >= gen:
                continue
            n = 1 if i % 2 == 0 else min(4, gen - pos[i])
            feeds.append(streams[i][pos[i] - 1:pos[i] - 1 + n])
            sess.append(snap[i])
            owners.append((i, n))
        ids, _ = model.step_ragged(sess, feeds, all_rows=True)
        at = 0
        for i, n in owners:
            assert [int(t) for t in ids[at:at + n]] == streams[i][pos[i]:pos[i] + n], (i, pos[i])
            pos[i] += n
            at += n
    # request 1 against the oracle: trunk + suffix, then its greedy stream
    oc = oracle.new_cache()
    ref = oracle.forward(np.concatenate([trunk, suffixes[1]]), oc)
    for k in range(gen):
        assert ora.argmax_first(ref) == streams[1][k], k
        if k + 1 < gen:
            ref = oracle.forward([streams[1][k]], oc)
    for s in reqs + snap + [root]:
        s.free()


def test_long_and_short_prefill_in_one_step(m35):
    """A 150-token and a 7-token sequence prefilled in one ragged step (the
    long one's GEMVs take whole 128-row GEMM blocks only through the batch),
    both against the oracle, then decode."""
    model, oracle = m35
    rng = np.random.default_rng(77)
    long_p, short_p = rng.integers(0, model.cfg.vocab, 150), rng.integers(0, model.cfg.vocab, 7)
    a, b = model.new_session(), model.new_session()
    _, logits = model.step_ragged([a, b], [long_p, short_p], want_logits=True)
    oa, ob = oracle.new_cache(), oracle.new_cache()
    ra, rb = oracle.forward(long_p, oa), oracle.forward(short_p, ob)
    assert rel(logits[0], ra) < LOGIT_TOL and rel(logits[1], rb) < LOGIT_TOL
    for step in range(4):
        t = ora.argmax_first(ra)
        assert ora.argmax_first(logits[0]) == t, step
        g, ra = a.forward([t]), oracle.forward([t], oa)
        assert rel(g, ra) < LOGIT_TOL, step
        logits = [g]
    a.free()
    b.free()


def test_continued_long_prefill(m35):
    """A 100-token prefill continued by a 90-token one and a 33-token one, so
    the long-row conv segments and the chunkwise recurrence start from a
    state that earlier steps wrote, against the oracle fed the same pieces."""
    model, oracle = m35
    rng = np.random.default_rng(78)
    a = model.new_session()
    oa = oracle.new_cache()
    for n in (100, 90, 33):
        toks = rng.integers(0, model.cfg.vocab, n)
        g, r = a.forward(toks), oracle.forward(toks, oa)
        assert rel(g, r) < LOGIT_TOL, n
    a.free()


def test_short_and_segmented_prefill_then_decode(m35):
    """A 2-token sequence (shorter than the conv history, so its new conv state
    mixes old state and inputs) prefilled in one step with a 140-token one
    (three 64-row conv segments, the chunkwise recurrence), after a first
    feed that left both with nonzero state; then both decode. Against the
    oracle fed the same pieces."""
    model, oracle = m35
    rng = np.random.default_rng(79)
    a, b = model.new_session(), model.new_session()
    oa, ob = oracle.new_cache(), oracle.new_cache()
    first = [rng.integers(0, model.cfg.vocab, 5), rng.integers(0, model.cfg.vocab, 3)]
    model.step_ragged([a, b], first)
    oracle.forward(first[0], oa)
    oracle.forward(first[1], ob)
    long_p, short_p = rng.integers(0, model.cfg.vocab, 140), rng.integers(0, model.cfg.vocab, 2)
    _, logits = model.step_ragged([a, b], [long_p, short_p], want_logits=True)
    ra, rb = oracle.forward(long_p, oa), oracle.forward(short_p, ob)
    assert rel(logits[0], ra) < LOGIT_TOL and rel(logits[1], rb) < LOGIT_TOL
    for step in range(3):
        ta, tb = ora.argmax_first(ra), ora.argmax_first(rb)
        _, logits = model.step_ragged([a, b], [[ta], [tb]], want_logits=True)
        ra, rb = oracle.forward([ta], oa), oracle.forward([tb], ob)
        assert rel(logits[0], ra) < LOGIT_TOL and rel(logits[1], rb) < LOGIT_TOL, step
    a.free()
    b.free()


def test_forty_row_steps_take_two_chunk_launches(m35):
    """40 sessions stepped together: a 120-row prefill (two 64- and 56-row
    launches) and 40-row decode steps, so the fused gate/up runs as stream-K
    launches of two 32-row activation chunks. Every session against the
    oracle fed the same tokens, and each step's greedy ids equal the oracle's."""
    model, oracle = m35
    rng = np.random.default_rng(80)
    n = 40
    sess = [model.new_session() for _ in range(n)]
    caches = [oracle.new_cache() for _ in range(n)]
    feeds = [rng.integers(0, model.cfg.vocab, 3) for _ in range(n)]
    for step in range(3):
        _, logits = model.step_ragged(sess, feeds, want_logits=True)
        refs = [oracle.forward(f, c) for f, c in zip(feeds, caches)]
        for i in range(n):
            assert rel(logits[i], refs[i]) < LOGIT_TOL, (step, i)
        feeds = [[ora.argmax_first(r)] for r in refs]
        assert [ora.argmax_first(l) for l in logits] == [f[0] for f in feeds], step
    for s in sess:
        s.free()
