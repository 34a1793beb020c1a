"""Captured decode steps (pgd_model_set_graphs): a step's launches replayed
from a HIP graph give bitwise the logits of the same steps launched eagerly,
for the hybrid model (Gated-DeltaNet + gated attention, A8) and Qwen2 (GGUF
k-quants in both arithmetics), across KV page boundaries and an attention
chunk boundary (a new launch signature mid-decode), for batch-1 greedy decode
(Qwen35::forward_greedy, pagoda-hf/src/qwen3_5.rs:505-529) and ragged
batched steps."""
import numpy as np
import pytest

from test_gpu_model import small2, small35

pytestmark = pytest.mark.gpu


def _decode(model, prompt, steps):
    s = model.new_session()
    out = [s.forward(prompt)]
    tok = int(np.argmax(out[-1]))
    for _ in range(steps):
        out.append(s.forward([tok]))
        tok = int(np.argmax(out[-1]))
    s.free()
    return np.stack(out)


@pytest.mark.parametrize("arch", ["qwen35", "qwen2_q8", "qwen2_f32"])
@pytest.mark.parametrize("plen", [11, 250])
def test_graph_replay_bitwise_equals_eager(dev, arch, plen):
    from pagoda_amd.engine import ARITH_DEQUANT_F32, Model

    print(f"graphs {arch} prompt {plen}", flush=True)
    cfg = small35() if arch == "qwen35" else small2()
    model = Model.synth(dev, cfg, 17)
    try:
        if arch == "qwen2_f32":
            model.set_kquant_arith(ARITH_DEQUANT_F32)
        prompt = np.random.default_rng(plen).integers(0, cfg.vocab, plen)
        steps = 12  # crosses a KV page; from 250 also the 256-position chunk
        eager = _decode(model, prompt, steps)
        model.set_graphs(True)
        graphed = _decode(model, prompt, steps)
        again = _decode(model, prompt, steps)
        st = model.graph_stats()
        assert st["replays"] >= steps, st
        np.testing.assert_array_equal(graphed.view(np.uint32), eager.view(np.uint32))
        np.testing.assert_array_equal(again.view(np.uint32), eager.view(np.uint32))
    finally:
        model.free()


def test_graph_ragged_batches_and_eager_work_between(dev):
    """Batched steps of 3 sessions (one of them feeding 4-token verify rows
    part of the time), replayed from graphs, with eager GEMV work and
    synchronizations between the replays: every step's ids and logits equal
    the eager run's."""
    from pagoda_amd import Matrix
    from pagoda_amd.engine import Model

    cfg = small35()
    model = Model.synth(dev, cfg, 23)
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, cfg.vocab, n) for n in (9, 30, 17)]
    plan = [[1, 1, 1], [1, 4, 1], [1, 1, 1], [1, 4, 1]] * 3
    side = Matrix.synth(dev, 0, 512, 256, 1, 1, 0.02)
    x = rng.normal(0, 1, (7, 256)).astype(np.float32)

    def run():
        ss = [model.new_session() for _ in prompts]
        ids, _ = model.step_ragged(ss, prompts)
        res = []
        for k, ns in enumerate(plan):
            feeds = [[int(ids[i])] + [int((ids[i] + j) % cfg.vocab) for j in range(1, n)] for i, n in enumerate(ns)]
            ids, lg = model.step_ragged(ss, feeds, want_logits=True)
            res.append(lg)
            side.gemv(x)  # eager launches on the same stream between replays
        for s in ss:
            s.free()
        return np.stack(res)

    try:
        eager = run()
        model.set_graphs(True)
        g1 = run()
        g2 = run()
        assert model.graph_stats()["replays"] > 0
        np.testing.assert_array_equal(g1.view(np.uint32), eager.view(np.uint32))
        np.testing.assert_array_equal(g2.view(np.uint32), eager.view(np.uint32))
    finally:
        side.free()
        model.free()
