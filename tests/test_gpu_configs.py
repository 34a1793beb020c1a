"""Full-size configurations against the CPU oracle on identical seeded weights.

Config 1: Qwen2.5-0.5B architecture, Q4_K_M-style
GGUF weights, 81-token random prompt, 32 greedy tokens; then the warm rerun
where the prefix graft slices the cold session to 80 prompt tokens and only
32 are fed
(pagoda/docs/BENCHMARK-METAL.md:25-33; examples/qwen2_gguf.rs:121-136: cold
and warm token streams are identical).

Config 4 widths on one 3:1 layer group: hidden 5120, SwiGLU
17408, 24/4 heads of 256, 16/32 GDN heads of 128, A8 weights.

The greedy rule is the engine sampler's (first max, pagoda/src/sampler.rs:59-69);
the top-2 logit margin of every step is printed so a near-tie is visible.
"""
import numpy as np
import pytest

from oracle import pyoracle as ora

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def rel(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def margin(x):
    t = np.sort(x)[-2:]
    return float(t[1] - t[0])


@pytest.mark.parametrize("arith", ["dequant_f32", "cpu_q8"])
def test_config1_qwen2_05b_greedy_32_cold_and_warm(dev, arith, capsys):
    """cpu_q8 (the Qwen2 default, the reference CPU path's arithmetic:
    candle's quantized matmul, qwen2_gguf.rs:280-289): every logit of the
    prompt and of 32 free-running greedy steps is bit-equal to the oracle's
    restatement, so the token streams are identical. dequant_f32 (f32
    dequant-then-dot, the Metal-like arithmetic) against the oracle in the
    same arithmetic: logits within 1e-3 and 32 identical greedy ids. Both:
    the warm rerun through the prefix graft reproduces the cold stream."""
    from pagoda_amd.engine import ARITH_CPU_Q8, ARITH_DEQUANT_F32, QWEN2_05B, Model, argmax_first

    cfg = QWEN2_05B
    seed = 1
    q8 = arith == "cpu_q8"
    mode = ARITH_CPU_Q8 if q8 else ARITH_DEQUANT_F32
    print("config1: building device model", flush=True)
    model = Model.synth(dev, cfg, seed)
    model.set_kquant_arith(mode)
    print("config1: building oracle model", flush=True)
    oracle = ora.Qwen2(ora.Qwen2Config(), seed, kquant_mode=mode)
    rng = np.random.default_rng(81)
    prompt = rng.integers(0, cfg.vocab, 81)
    s = model.new_session()
    oc = oracle.new_cache()
    got = s.forward(prompt)
    ref = oracle.forward(prompt, oc)
    gen_gpu, margins = [], []
    for step in range(32):
        if q8:
            np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32), err_msg=f"step {step}")
        else:
            assert rel(got, ref) < LOGIT_TOL, f"step {step}: {rel(got, ref)}"
        tg, tr = argmax_first(got), ora.argmax_first(ref)
        margins.append(margin(ref))
        assert tg == tr, f"step {step}: gpu {tg} oracle {tr} (margin {margins[-1]:.3g})"
        gen_gpu.append(tg)
        if step == 31:
            break
        got = s.forward([tg])
        ref = oracle.forward([tr], oc)
    with capsys.disabled():
        print(f"\n[config1 {arith}] 32 greedy ids equal; min top-2 margin {min(margins):.4g}", flush=True)
    s.free()
    # warm rerun: graft_session(prompt, len - 1) slices a cold session's
    # cache (81 prompt + 31 generated positions) to the 80 covered prompt
    # tokens (pagoda-hf/src/lib.rs:603-616); it feeds the last prompt token,
    # then the 31 tokens it samples itself
    cold = model.new_session()
    lg = cold.forward(prompt)
    for t in gen_gpu[:31]:
        assert argmax_first(lg) == t
        lg = cold.forward([t])
    assert cold.context_len() == 112
    w2 = cold.fork_prefix(80)
    assert w2.context_len() == 80
    fed = 0
    logits = w2.forward(prompt[80:])
    fed += 1
    warm_ids = []
    for step in range(32):
        t = argmax_first(logits)
        warm_ids.append(t)
        if step == 31:
            break
        logits = w2.forward([t])
        fed += 1
    assert fed == 32
    assert warm_ids == gen_gpu


def test_config4_widths_one_layer_group(dev):
    from pagoda_amd.engine import QWEN35_27B, Model, argmax_first
    from dataclasses import replace

    cfg = replace(QWEN35_27B, n_layers=4, vocab=32768, max_pos=256, kv_blocks=64)
    seed = 4
    model = Model.synth(dev, cfg, seed)
    oracle = ora.Qwen35(ora.Qwen35Config(n_layers=4, vocab=32768), seed)
    rng = np.random.default_rng(19)
    prompt = rng.integers(0, cfg.vocab, 19)
    s = model.new_session()
    oc = oracle.new_cache()
    got = s.forward(prompt)
    ref = oracle.forward(prompt, oc)
    assert rel(got, ref) < LOGIT_TOL
    for step in range(8):
        assert argmax_first(got) == ora.argmax_first(ref), step
        t = ora.argmax_first(ref)
        got = s.forward([t])
        ref = oracle.forward([t], oc)
        assert rel(got, ref) < LOGIT_TOL, (step, rel(got, ref))


def _elementwise_ok(got, ref, tol=1e-3):
    """|d| <= tol*|ref| + atol per logit, atol = 0.1 * tol * max|ref|."""
    g, r = got.astype(np.float64), ref.astype(np.float64)
    return bool(np.all(np.abs(g - r) <= tol * np.abs(r) + 0.1 * tol * np.abs(r).max()))


def test_config4_full_depth_greedy_32_and_batch32(dev, capsys):
    """Config 4 at full size (64 layers, vocab 151936) against the oracle on
    the same seeded weights: 19-token prompt, 32 greedy tokens at batch 1,
    logits within 1e-3 at every step (the reference's own check,
    examples/qwen3_8.rs:219-247, 314-326). Then one batch-32 decode step
    whose rows equal their batch-1 counterparts within the 1e-5 class with
    the same greedy ids."""
    import time
    from dataclasses import replace

    from pagoda_amd.engine import QWEN35_27B, Model, argmax_first

    def say(msg):
        with capsys.disabled():
            print(f"\n[config4 full depth] {msg}", flush=True)

    cfg = replace(QWEN35_27B, max_pos=512, kv_blocks=256)
    seed = 4
    t0 = time.time()
    model = Model.synth(dev, cfg, seed)
    say(f"device model built ({time.time() - t0:.1f} s)")
    oracle = ora.Qwen35(ora.Qwen35Config(), seed)
    say(f"oracle model built ({time.time() - t0:.1f} s, {ora.lib().ora_num_threads()} threads)")
    prompt = np.random.default_rng(19).integers(0, cfg.vocab, 19)
    s = model.new_session()
    oc = oracle.new_cache()
    got, ref = s.forward(prompt), oracle.forward(prompt, oc)
    margins = []
    for step in range(32):
        assert rel(got, ref) < LOGIT_TOL, (step, rel(got, ref))
        assert _elementwise_ok(got, ref), step
        tg, tr = argmax_first(got), ora.argmax_first(ref)
        margins.append(margin(ref))
        assert tg == tr, f"step {step}: gpu {tg} oracle {tr} (margin {margins[-1]:.3g})"
        if step == 31:
            break
        got, ref = s.forward([tg]), oracle.forward([tr], oc)
        if step % 8 == 7:
            say(f"step {step + 1}/32 equal ({time.time() - t0:.1f} s)")
    say(f"32 greedy ids equal, min top-2 margin {min(margins):.4g}")
    s.free()
    # batch 32: distinct prompts, then one decode step batched vs alone. The
    # 32-row launches take other kernels (split-K shared-operand, stream-K)
    # than 1-row launches; each is within fp32 rounding of the other per
    # layer, which over 64 layers stays below 1e-4 of the logits' scale.
    rng = np.random.default_rng(32)
    prompts = [rng.integers(0, cfg.vocab, 19) for _ in range(32)]
    sess = [model.new_session() for _ in range(32)]
    ids, _ = model.step_ragged(sess, prompts)
    alone = [x.fork() for x in sess]
    feed = [[int(t)] for t in ids]
    bid, blog = model.step_ragged(sess, feed, want_logits=True)
    worst = 0.0
    for i in range(32):
        lg = alone[i].forward(feed[i])
        worst = max(worst, rel(blog[i], lg))
        assert rel(blog[i], lg) < 1e-4, i
        assert int(bid[i]) == argmax_first(lg), i
    say(f"batch-32 rows vs batch 1: max rel {worst:.2e}")
    # two batch-32 rows against the oracle
    for i in (0, 31):
        c = oracle.new_cache()
        r = oracle.forward(prompts[i], c)
        assert ora.argmax_first(r) == int(ids[i]), i
        r = oracle.forward(feed[i], c)
        assert rel(blog[i], r) < LOGIT_TOL and _elementwise_ok(blog[i], r), i
        assert ora.argmax_first(r) == int(bid[i]), i
    for x in sess + alone:
        x.free()
    model.free()
    say(f"batch-32 step checked ({time.time() - t0:.1f} s)")


def test_config4_widths_prefill_300_tokens(dev):
    """A 300-token prompt at config-4 widths (one 3:1 layer group) is
    prefilled through the A8 GEMM (weights read once per 128 rows) and the
    GEMM path's prepared-output emits; logits against the oracle within 1e-3,
    then 4 greedy decode steps."""
    from dataclasses import replace

    from pagoda_amd.engine import QWEN35_27B, Model, argmax_first

    cfg = replace(QWEN35_27B, n_layers=4, vocab=32768, max_pos=512, kv_blocks=64)
    seed = 6
    model = Model.synth(dev, cfg, seed)
    oracle = ora.Qwen35(ora.Qwen35Config(n_layers=4, vocab=32768), seed)
    prompt = np.random.default_rng(300).integers(0, cfg.vocab, 300)
    s = model.new_session()
    oc = oracle.new_cache()
    got = s.forward(prompt)
    ref = oracle.forward(prompt, oc)
    assert rel(got, ref) < LOGIT_TOL and _elementwise_ok(got, ref)
    for step in range(4):
        assert argmax_first(got) == ora.argmax_first(ref), step
        t = ora.argmax_first(ref)
        got, ref = s.forward([t]), oracle.forward([t], oc)
        assert rel(got, ref) < LOGIT_TOL, (step, rel(got, ref))
    s.free()
    model.free()


def _c5_passes(model, trunk, suffixes, gen, want_logits=False):
    """Config-5 pattern: every request forks one
    prefilled trunk (KV pages shared copy-on-write), its suffix is prefilled
    in one ragged step, then pass A decodes one token per request per step;
    pass B restarts from the same post-suffix states and packs 1-token decode
    rows (even requests) with 4-token known-token verify chunks (odd
    requests, replaying pass A's tokens) into one ragged batch per step.
    Returns pass A's streams (and logits per step) and the number of verified
    ids that differ from pass A's."""
    root = model.new_session()
    root.forward(trunk)
    reqs = [root.fork() for _ in suffixes]
    first, lg = model.step_ragged(reqs, suffixes, want_logits=want_logits)
    logits = [lg]
    snap = [r.fork() for r in reqs]
    streams = [[int(t)] for t in first]
    for _ in range(gen - 1):
        ids, lg = model.step_ragged(reqs, [[s[-1]] for s in streams], want_logits=want_logits)
        logits.append(lg)
        for s, t in zip(streams, ids):
            s.append(int(t))
    n = len(suffixes)
    pos = [1] * n
    mismatches = 0
    while any(p < gen for p in pos):
        sess, feeds, owners = [], [], []
        for i in range(n):
            if pos[i] >= gen:
                continue
            k = 1 if i % 2 == 0 else min(4, gen - pos[i])
            feeds.append(streams[i][pos[i] - 1:pos[i] - 1 + k])
            sess.append(snap[i])
            owners.append((i, k))
        ids, _ = model.step_ragged(sess, feeds, all_rows=True)
        at = 0
        for i, k in owners:
            mismatches += sum(int(t) != s for t, s in zip(ids[at:at + k], streams[i][pos[i]:pos[i] + k]))
            pos[i] += k
            at += k
    for s in reqs + snap + [root]:
        s.free()
    return streams, logits, mismatches


def test_config5_widths_shared_trunk_mixed_verify(dev, capsys):
    """Config 5 at config-4 widths on one 3:1 layer group (reduced vocab): a
    300-token trunk (two 256-position attention chunks, so every row's
    attention merges chunks) shared by 64 forks with distinct 50-token
    suffixes; 64-row decode steps (two-chunk launches) and mixed decode /
    verify batches. Every verified id equals the decoded stream, and two
    requests' logits at every step are within 1e-3 of the oracle fed the same
    tokens, with the oracle's greedy ids."""
    import time
    from dataclasses import replace

    from pagoda_amd.engine import QWEN35_27B, Model

    cfg = replace(QWEN35_27B, n_layers=4, vocab=8192, max_pos=512, kv_blocks=2048)
    seed = 55
    t0 = time.time()
    model = Model.synth(dev, cfg, seed)
    rng = np.random.default_rng(300)
    trunk = rng.integers(0, cfg.vocab, 300)
    suffixes = [rng.integers(0, cfg.vocab, 50) for _ in range(64)]
    gen = 8
    streams, logits, mism = _c5_passes(model, trunk, suffixes, gen, want_logits=True)
    with capsys.disabled():
        print(f"\n[config5 widths] gpu passes done ({time.time() - t0:.1f} s), verify mismatches {mism}", flush=True)
    assert mism == 0
    oracle = ora.Qwen35(ora.Qwen35Config(n_layers=4, vocab=cfg.vocab), seed)
    oc = oracle.new_cache()
    oracle.forward(trunk, oc)
    for i in (0, 37):
        c = oc.clone()
        ref = oracle.forward(suffixes[i], c)
        for k in range(gen):
            got = logits[k][i]
            assert rel(got, ref) < LOGIT_TOL, (i, k, rel(got, ref))
            assert ora.argmax_first(ref) == streams[i][k], (i, k, margin(ref))
            if k + 1 < gen:
                ref = oracle.forward([streams[i][k]], c)
    with capsys.disabled():
        print(f"[config5 widths] oracle checks done ({time.time() - t0:.1f} s)", flush=True)
    model.free()


def test_config5_full_size_verify_is_exact(dev, capsys):
    """Config 5 at full size (64 layers, vocab 151936): 64 requests share one
    3968-token trunk, add 50-token suffixes and decode; every token a 4-token
    verify chunk yields in the mixed pass equals the decode pass's token
    (the size-independent property the continuous-batching engine relies on
    when it accepts verified tokens)."""
    import time
    from dataclasses import replace

    from pagoda_amd.engine import QWEN35_27B, Model

    trunk_len, sfx, gen = 3968, 50, 9
    cfg = replace(QWEN35_27B, max_pos=4096 + 64,
                  kv_blocks=(trunk_len // 16 + 2) + 2 * 64 * ((sfx + gen + 4) // 16 + 2) + 16)
    t0 = time.time()
    model = Model.synth(dev, cfg, 2026)
    rng = np.random.default_rng(5)
    trunk = rng.integers(0, cfg.vocab, trunk_len)
    suffixes = [rng.integers(0, cfg.vocab, sfx) for _ in range(64)]
    streams, _, mism = _c5_passes(model, trunk, suffixes, gen)
    with capsys.disabled():
        print(f"\n[config5 full size] {time.time() - t0:.1f} s, verify mismatches {mism}", flush=True)
    assert mism == 0
    assert all(len(s) == gen for s in streams)
    model.free()
