"""Pins the oracle's restatement of candle's CPU k-quant matmul
(pagoda-hf/src/qwen2_gguf.rs:280-289 keeps QMatMul on the CPU; candle-core
0.8.4 quantizes each activation row to Q8_K and takes integer block dots):
Q8_K quantization known answers, the block dots against hand-built blocks
and against the fp64 value of the same integers, and the model-level switch."""
import numpy as np

from oracle import pyoracle as ora
from test_oracle_formats import _q4k_block


def test_q8k_quantize_known_answers():
    x = np.arange(1, 257, dtype=np.float32)  # max 256 -> iscale -0.5
    b = ora.q8k_quantize(x)[0]
    assert b["d"] == np.float32(-2.0)
    # round half away from zero: -0.5 -> -1, -1.5 -> -2, ..., -128 at the max
    want = -((np.arange(1, 257) + 1) // 2)
    np.testing.assert_array_equal(b["qs"], want)
    np.testing.assert_array_equal(b["bsums"], want.reshape(16, 16).sum(1))
    # the first |max| wins; the opposite extreme saturates at +127
    x = np.zeros(256, np.float32)
    x[3], x[9] = 4.0, -4.0
    b = ora.q8k_quantize(x)[0]
    assert b["d"] == np.float32(-1.0 / 32) and b["qs"][3] == -128 and b["qs"][9] == 127
    # an all-zero block
    b = ora.q8k_quantize(np.zeros(256, np.float32))[0]
    assert b["d"] == 0 and not b["qs"].any() and not b["bsums"].any()
    # a 320-wide row: the tail of the second block is zero-padded
    x = np.random.default_rng(0).normal(0, 1, 320).astype(np.float32)
    q = ora.q8k_quantize(x)
    assert q.size == 2 and not q[1]["qs"][64:].any()
    np.testing.assert_allclose(q[0]["d"] * q[0]["qs"], x[:256], atol=abs(q[0]["d"]) / 2 + 1e-7)


def _q8k(d, qs):
    qs = np.asarray(qs, np.int8)
    b = np.zeros(1, ora.Q8K_DTYPE)
    b["d"], b["qs"], b["bsums"] = d, qs, qs.astype(np.int32).reshape(16, 16).sum(1)
    return b


def test_q4k_q8k_dot_hand_built():
    ones = [0x11] * 128  # every nibble 1
    blk = _q4k_block(1.0, 0.0, [1] * 8, [0] * 8, ones)
    assert ora.kq_vec_dot_q8k(1, blk, 1, 256, _q8k(1.0, [1] * 256))[0] == 256.0
    # the min term subtracts dmin * m * sum(q8): 256 - 256 = 0
    blk = _q4k_block(1.0, 1.0, [1] * 8, [1] * 8, ones)
    assert ora.kq_vec_dot_q8k(1, blk, 1, 256, _q8k(1.0, [1] * 256))[0] == 0.0
    # sub-block j scale j+1 against q8 = 1 on sub-block 5 only (elements
    # 160..191 = high nibbles of bytes 64..95): 32 * 6 * 1
    q = np.zeros(256, np.int8)
    q[160:192] = 1
    blk = _q4k_block(1.0, 0.0, list(range(1, 9)), [0] * 8, ones)
    assert ora.kq_vec_dot_q8k(1, blk, 1, 256, _q8k(0.5, q))[0] == 32 * 6 * 0.5


def _fp64_dot(deq, q8k, n_in):
    xq = np.concatenate([b["d"].astype(np.float64) * b["qs"].astype(np.float64) for b in q8k])[:n_in]
    return deq.astype(np.float64) @ xq


def test_kq_q8k_dot_equals_fp64_of_the_integers():
    """vec_dot == sum_i dequant(w)_i * d8 * q8_i: the same integers in fp64
    (any index, nibble-half, qh-plane or scale slip fails this)."""
    rng = np.random.default_rng(3)
    for n_in in (256, 896, 1024):
        w = rng.normal(0, 0.02, (24, n_in)).astype(np.float32)
        x = rng.normal(0, 1, n_in).astype(np.float32)
        q8 = ora.q8k_quantize(x)
        for fmt, quant, deq in ((1, ora.q4k_quantize, ora.q4k_dequant), (2, ora.q6k_quantize, ora.q6k_dequant)):
            blk = quant(w)
            got = ora.kq_vec_dot_q8k(fmt, blk, 24, n_in, q8)
            ref = _fp64_dot(deq(blk, 24, n_in), q8, n_in)
            np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5 * np.abs(ref).max())
            # and within Q8_K's quantization error of the f32 activations
            exact = deq(blk, 24, n_in).astype(np.float64) @ x.astype(np.float64)
            assert np.abs(got - exact).max() < 2e-2 * np.abs(exact).max()


def test_model_switch_to_q8k_mode():
    cfg = ora.Qwen2Config(n_layers=2, hidden=256, intermediate=512, vocab=512, heads=4, kv_heads=2, head_dim=64,
                          max_pos=64, rope_theta=1e6, eps=1e-6)
    m = ora.Qwen2(cfg, 9, kquant_mode=0)
    a = m.forward([1, 2, 3], m.new_cache())
    m.set_kquant_mode(1)
    b = m.forward([1, 2, 3], m.new_cache())
    m.set_kquant_mode(0)
    c = m.forward([1, 2, 3], m.new_cache())
    np.testing.assert_array_equal(a, c)
    assert not np.array_equal(a, b)
    assert np.abs(a - b).max() < 0.05 * np.abs(a).max()


# ------------------------------------------------ Q8_0 activations (32-weight types)
def test_q8_0_activation_known_answers():
    # amax 127 -> d = 1, id = 1: q = round(x), halves away from zero
    x = np.zeros(32, np.float32)
    x[:8] = [0.5, 1.5, 2.5, -0.5, -2.5, 126.49, -3.5, 127.0]
    b = ora.q8_0_quantize_act(x)[0]
    assert b["d"] == np.float16(1.0).view(np.uint16)
    np.testing.assert_array_equal(b["qs"][:8], [1, 2, 3, -1, -3, 126, -4, 127])
    # d = amax / 127 stored as f16; an all-zero block has d 0 and q 0
    x = np.concatenate([np.full(32, 2.54, np.float32), np.zeros(32, np.float32)])
    q = ora.q8_0_quantize_act(x)
    assert q[0]["d"] == np.float16(np.float32(2.54) / np.float32(127)).view(np.uint16)
    assert (q[0]["qs"] == 127).all() and q[1]["d"] == 0 and not q[1]["qs"].any()


def test_q8_0_q5_0_dots():
    from test_oracle_formats import q5_0_block, q8_0_block

    w = np.frombuffer(q8_0_block(0.5, [2] * 32), np.uint8)
    act = np.zeros(1, ora.Q8_0_ACT_DTYPE)
    act["d"], act["qs"] = np.float16(1.0).view(np.uint16), 3
    assert ora.q8_0_vec_dot(3, w, 1, 32, act)[0] == 96.0
    j = np.arange(16)
    w5 = np.frombuffer(q5_0_block(1.0, 0xFFFF0000, j | (j << 4)), np.uint8)  # weights 0..31 -> -16..15
    act["qs"] = 1
    assert ora.q8_0_vec_dot(4, w5, 1, 32, act)[0] == float(np.arange(32).sum() - 16 * 32)
    # random blocks: the dot equals the fp64 value of the same integers
    from checkpoints import GGML_Q5_0, GGML_Q8_0, random_blocks

    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, 320).astype(np.float32)
    q8 = ora.q8_0_quantize_act(x)
    xq = np.concatenate([np.float16(0).view(np.uint16).dtype.type(b["d"]).view(np.float16).astype(np.float64)
                         * b["qs"].astype(np.float64) for b in q8])
    for fmt, gt, deq in ((3, GGML_Q8_0, ora.q8_0_dequant), (4, GGML_Q5_0, ora.q5_0_dequant)):
        blk = random_blocks(rng, gt, 16, 320, d_std=0.01)
        got = ora.q8_0_vec_dot(fmt, blk, 16, 320, q8)
        ref = deq(blk, 16, 320).astype(np.float64) @ xq
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
