"""Models loaded from checkpoint files: an MLX directory (Qwen35::load,
qwen3_5.rs:338-452) and a Qwen2 GGUF file (qwen2_gguf.rs:65-140), written
from the oracle's seeded weights. With the synthetic generator's values the
loaded model must equal Model.synth bit for bit; with every norm weight
perturbed it must match the oracle, which pins which file tensor lands in
which slot."""
import numpy as np
import pytest

from checkpoints import (gguf_tensors_from_oracle, mlx_tensors_from_oracle, mlx_text_config, perturb_norms_qwen2,
                         perturb_norms_qwen35, qwen2_meta, write_gguf, write_mlx_config, write_safetensors_shards)
from test_gpu_model import LOGIT_TOL, oracle2, oracle35, rel, small2, small35

pytestmark = pytest.mark.gpu


def greedy_logits(model, prompt, steps):
    """Logits of the prompt and of `steps` greedy decode steps."""
    s = model.new_session()
    try:
        out = [s.forward(prompt)]
        for _ in range(steps):
            out.append(s.forward([int(np.argmax(out[-1]))]))
        return out
    finally:
        s.free()


def oracle_logits(oracle, prompt, steps):
    c = oracle.new_cache()
    out = [oracle.forward(prompt, c)]
    for _ in range(steps):
        out.append(oracle.forward([int(np.argmax(out[-1]))], c))
    return out


def mlx_checkpoint(tmp_path, cfg, oracle):
    d = tmp_path / "mlx"
    write_mlx_config(d, mlx_text_config(cfg, max_pos=cfg.max_pos))
    write_safetensors_shards(d, mlx_tensors_from_oracle(cfg, oracle), nshards=3)
    return d


def test_mlx_checkpoint_equals_synthetic_model(dev, tmp_path):
    from pagoda_amd.engine import Model

    cfg = small35(n_layers=4)
    d = mlx_checkpoint(tmp_path, cfg, oracle35(cfg, 11))
    loaded = Model.load_mlx(dev, d, kv_blocks=cfg.kv_blocks)
    synth = Model.synth(dev, cfg, 11)
    try:
        assert loaded.cfg.full_every == cfg.full_every and loaded.cfg.rotary_dim == cfg.rotary_dim
        prompt = np.random.default_rng(5).integers(0, cfg.vocab, 9)
        for a, b in zip(greedy_logits(loaded, prompt, 6), greedy_logits(synth, prompt, 6)):
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        loaded.free()
        synth.free()


def test_mlx_checkpoint_norms_match_oracle(dev, tmp_path):
    from pagoda_amd.engine import Model

    cfg = small35(n_layers=4)
    oracle = oracle35(cfg, 12)
    perturb_norms_qwen35(cfg, oracle, np.random.default_rng(1))
    d = mlx_checkpoint(tmp_path, cfg, oracle)
    loaded = Model.load_mlx(dev, d, kv_blocks=cfg.kv_blocks)
    try:
        prompt = np.random.default_rng(6).integers(0, cfg.vocab, 7)
        got, ref = greedy_logits(loaded, prompt, 6), oracle_logits(oracle, prompt, 6)
        for step, (a, b) in enumerate(zip(got, ref)):
            assert rel(a, b) < LOGIT_TOL, f"step {step}: {rel(a, b)}"
            assert int(np.argmax(a)) == int(np.argmax(b)), f"greedy token diverged at step {step}"
    finally:
        loaded.free()


def test_mlx_missing_tensor_is_an_error(dev, tmp_path):
    from pagoda_amd._lib import PagodaError
    from pagoda_amd.engine import Model

    cfg = small35(n_layers=4)
    tensors = mlx_tensors_from_oracle(cfg, oracle35(cfg, 11))
    del tensors["language_model.model.layers.2.linear_attn.in_proj_b.biases"]
    d = tmp_path / "mlx"
    write_mlx_config(d, mlx_text_config(cfg, max_pos=cfg.max_pos))
    write_safetensors_shards(d, tensors)
    with pytest.raises(PagodaError) as e:
        Model.load_mlx(dev, d, kv_blocks=cfg.kv_blocks)
    assert e.value.code == -7 and "layers.2.linear_attn.in_proj_b.biases" in str(e.value)


def q2cfg():
    # K-quant rows of whole super-blocks: hidden and intermediate multiples of 256
    return small2(intermediate=512)


@pytest.mark.parametrize("untied", [False, True])
def test_gguf_checkpoint_equals_synthetic_model(dev, tmp_path, untied):
    from pagoda_amd.engine import Model

    cfg = q2cfg()
    p = tmp_path / "q2.gguf"
    write_gguf(p, qwen2_meta(cfg), gguf_tensors_from_oracle(cfg, oracle2(cfg, 5), untied=untied))
    loaded = Model.load_gguf(dev, p, kv_blocks=cfg.kv_blocks)
    synth = Model.synth(dev, cfg, 5)
    try:
        assert loaded.cfg.intermediate == cfg.intermediate and loaded.cfg.vocab == cfg.vocab
        prompt = np.random.default_rng(7).integers(0, cfg.vocab, 11)
        for a, b in zip(greedy_logits(loaded, prompt, 6), greedy_logits(synth, prompt, 6)):
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        loaded.free()
        synth.free()


def test_gguf_checkpoint_norms_match_oracle(dev, tmp_path):
    from pagoda_amd.engine import Model

    cfg = q2cfg()
    oracle = oracle2(cfg, 6)
    perturb_norms_qwen2(cfg, oracle, np.random.default_rng(2))
    p = tmp_path / "q2.gguf"
    write_gguf(p, qwen2_meta(cfg), gguf_tensors_from_oracle(cfg, oracle))
    loaded = Model.load_gguf(dev, p, kv_blocks=cfg.kv_blocks)
    try:
        prompt = np.random.default_rng(8).integers(0, cfg.vocab, 9)
        got, ref = greedy_logits(loaded, prompt, 6), oracle_logits(oracle, prompt, 6)
        for step, (a, b) in enumerate(zip(got, ref)):
            assert rel(a, b) < LOGIT_TOL, f"step {step}: {rel(a, b)}"
            assert int(np.argmax(a)) == int(np.argmax(b)), f"greedy token diverged at step {step}"
    finally:
        loaded.free()
