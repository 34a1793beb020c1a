"""Pins the oracle's format code (A8 / Q4_K / Q6_K, fp16/bf16, generator)
against known answers that a plausible layout or rounding mistake fails."""
import numpy as np
import pytest

from oracle import pyoracle as ora


# ---------------------------------------------------------------- fp helpers
def test_bf16_round_trip_matches_reference_rule():
    # pagoda-hf/src/qwen3_gemv.rs:570-574: bits + 0x7fff + lsb, >> 16.
    # -0.24705882 has bits 0xbe7cfcfd -> 0xbe7d (the MLX vector's scale).
    assert ora.f32_to_bf16(-0.24705882370471954) == 0xBE7D
    assert ora.bf16_to_f32(0xBE7D) == np.float32(-0.2470703125)
    # exact ties round to even
    assert ora.f32_to_bf16(np.float32(1.0 + 2.0 ** -8)) == 0x3F80  # tie, lsb 0 -> down
    assert ora.f32_to_bf16(np.float32(1.0 + 3 * 2.0 ** -8)) == 0x3F82  # tie, lsb 1 -> up


def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.normal(0, 1, 2000), rng.normal(0, 1e-5, 500), rng.normal(0, 3e4, 200),
                         [0.0, -0.0, 65504.0, 65520.0, 1e-8, 5.96e-8, 6.1e-5]]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16)
    for x, r in zip(xs, ref):
        h = ora.f32_to_f16(float(x))
        assert h == int(r.view(np.uint16)), x
        assert ora.f16_to_f32(h) == np.float32(r), x


# ---------------------------------------------------------------- MLX A8
def test_mlx_affine_vector():
    """pagoda-hf/src/qwen3_5.rs:1760-1777: mx.quantize(arange(64)) gives the
    packed word 4093115391, scale bf16(-0.24705882), bias 63."""
    w = np.arange(64, dtype=np.float32).reshape(1, 64)
    packed, scales, biases = ora.a8_quantize(w)
    assert int(packed[0]) == 4093115391
    assert int(scales[0]) == ora.f32_to_bf16(-0.24705882370471954)
    assert ora.bf16_to_f32(int(biases[0])) == 63.0
    deq = ora.a8_dequant(packed, scales, biases, 1, 64)
    # The reference asserts 1e-3 against [0, .988, 1.976, 2.965] but with the
    # bf16-rounded scale code 255 gives 63 - 0.2470703*255 = -0.0029297, so
    # the formula value is reproduced exactly and the stated values to 3e-3.
    assert deq[0, 0] == np.float32(63.0) + np.float32(-0.2470703125) * np.float32(255)
    np.testing.assert_allclose(deq[0, :4], [0.0, 0.98823525, 1.9764705, 2.9647057], atol=3e-3)


def test_a8_dequant_closed_form_reference_patterns():
    """qwen3_gemv.rs:1038-1058 pattern: code = i % 256, scale .5, bias -1."""
    n_in = 256
    codes = (np.arange(n_in) % 256).astype(np.uint8)
    packed = codes.view(np.uint32)
    sc = np.full(n_in // 64, ora.f32_to_bf16(0.5), np.uint16)
    bi = np.full(n_in // 64, ora.f32_to_bf16(-1.0), np.uint16)
    deq = ora.a8_dequant(packed, sc, bi, 1, n_in)
    np.testing.assert_array_equal(deq[0], -1.0 + 0.5 * codes.astype(np.float32))
    # little-endian byte order inside the u32 word (0x01020304 -> 4,3,2,1)
    packed = np.full(64, 0x01020304, np.uint32)
    deq = ora.a8_dequant(packed, sc, np.full(4, 0, np.uint16), 1, 256)
    np.testing.assert_array_equal(deq[0, :4], [2.0, 1.5, 1.0, 0.5])


def test_a8_quantize_error_bound():
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, (7, 320)).astype(np.float32)
    packed, sc, bi = ora.a8_quantize(w)
    deq = ora.a8_dequant(packed, sc, bi, 7, 320)
    # codes round to half a step; storing the scale as bf16 (half ulp is up
    # to 2^-8 relative, times codes up to 255) adds up to ~one step, and the
    # bf16 bias up to 2^-8 |bias|
    g = w.reshape(7, 5, 64)
    step = (g.max(-1) - g.min(-1)) / 255
    err = np.abs(deq.reshape(7, 5, 64) - g).max(-1)
    assert np.all(err <= step * (0.5 + 255 * 2.0 ** -8) * 1.01 + np.abs(g).max(-1) * 2 ** -8)
    assert np.median(err / step) < 1.0


# ---------------------------------------------------------------- GGML Q4_K
def _q4k_block(d, dmin, sc, m, qs):
    """Assemble block_q4_K bytes by the public layout (independent packing)."""
    b = bytearray(144)
    b[0:2] = np.float16(d).tobytes()
    b[2:4] = np.float16(dmin).tobytes()
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] |= sc[j] & 63
            s[j + 4] |= m[j] & 63
        else:
            s[j + 4] |= (sc[j] & 15) | ((m[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    b[4:16] = bytes(s)
    b[16:144] = bytes(qs)
    return np.frombuffer(bytes(b), np.uint8)


def test_q4k_known_answers():
    # sub-block scales/mins chosen so a swapped index or nibble half shows
    sc = [1, 2, 3, 4, 33, 40, 50, 63]
    m = [5, 6, 7, 8, 17, 31, 48, 62]
    qs = [(i * 7 + 3) & 0xFF for i in range(128)]
    blk = _q4k_block(0.5, 0.25, sc, m, qs)
    deq = ora.q4k_dequant(blk, 1, 256)[0]
    # element 0: low nibble of qs[0] in sub-block 0
    assert deq[0] == 0.5 * 1 * (qs[0] & 15) - 0.25 * 5
    # element 32: high nibble of qs[0], sub-block 1
    assert deq[32] == 0.5 * 2 * (qs[0] >> 4) - 0.25 * 6
    # element 64+5: low nibble of qs[32+5], sub-block 2
    assert deq[69] == 0.5 * 3 * (qs[37] & 15) - 0.25 * 7
    # element 128+31: sub-block 4 (6-bit scale split across bytes), qs[64+31] low
    assert deq[159] == 0.5 * 33 * (qs[95] & 15) - 0.25 * 17
    # element 255: sub-block 7 high nibble of qs[127]
    assert deq[255] == 0.5 * 63 * (qs[127] >> 4) - 0.25 * 62
    # full closed form
    exp = np.zeros(256, np.float32)
    for e in range(256):
        j, l = divmod(e, 64)
        q = qs[32 * j + (l % 32)]
        nib = (q & 15) if l < 32 else (q >> 4)
        sb = 2 * j + (l >= 32)
        exp[e] = np.float32(np.float32(0.5) * sc[sb]) * nib - np.float32(np.float32(0.25) * m[sb])
    np.testing.assert_array_equal(deq, exp)


def test_q4k_tail_padding_k896():
    rng = np.random.default_rng(2)
    w = rng.normal(0, 0.02, (3, 896)).astype(np.float32)
    blk = ora.q4k_quantize(w)
    assert blk.size == 3 * 4 * 144
    deq = ora.q4k_dequant(blk, 3, 896)
    step = np.abs(w).max() * 2 / 15
    assert np.abs(deq - w).max() < step


def test_q4k_exact_grid_round_trip():
    # weights already on a Q4_K grid with 6-bit scales reproduce exactly
    d, dmin = 2.0 ** -6, 2.0 ** -7
    sc = [63, 32, 16, 8, 63, 1, 5, 40]
    mm = [63, 0, 12, 3, 7, 63, 1, 2]
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, 256)
    q[0:32:7] = 15  # make each sub-block hit both ends
    q[1:32:9] = 0
    w = np.zeros(256, np.float32)
    for e in range(256):
        sb = e // 32
        w[e] = np.float32(d * sc[sb]) * q[e] - np.float32(dmin * mm[sb])
    deq = ora.q4k_dequant(ora.q4k_quantize(w.reshape(1, 256)), 1, 256)[0]
    np.testing.assert_allclose(deq, w, atol=d * 64 * 0.51)


# ---------------------------------------------------------------- GGML Q6_K
def test_q6k_known_answers():
    ql = [(i * 13 + 1) & 0xFF for i in range(128)]
    qh = [(i * 29 + 7) & 0xFF for i in range(64)]
    sc = [(-1) ** i * (i + 1) * 3 for i in range(16)]
    d = 0.125
    b = bytearray(210)
    b[0:128] = bytes(ql)
    b[128:192] = bytes(qh)
    b[192:208] = np.array(sc, np.int8).tobytes()
    b[208:210] = np.float16(d).tobytes()
    deq = ora.q6k_dequant(np.frombuffer(bytes(b), np.uint8), 1, 256)[0]
    exp = np.zeros(256, np.float32)
    for e in range(256):
        n, r = divmod(e, 128)
        quad, l = divmod(r, 32)  # quad 0..3 -> (ql low, ql+32 low, ql high, ql+32 high)
        lq = ql[64 * n + l + (32 if quad in (1, 3) else 0)]
        nib = (lq & 15) if quad < 2 else (lq >> 4)
        hb = (qh[32 * n + l] >> (2 * quad)) & 3
        q = (nib | (hb << 4)) - 32
        s = sc[8 * n + 2 * quad + l // 16]
        exp[e] = np.float32(np.float32(d) * np.float32(s)) * np.float32(q)
    np.testing.assert_array_equal(deq, exp)


def test_q6k_quantize_error_bound():
    rng = np.random.default_rng(4)
    w = rng.normal(0, 0.02, (5, 896)).astype(np.float32)
    deq = ora.q6k_dequant(ora.q6k_quantize(w), 5, 896)
    g = w.reshape(5, -1, 16)
    step = np.abs(g).max(-1, keepdims=True) / 31
    err = np.abs(deq.reshape(5, -1, 16) - g)
    # half step of the per-16 scale, plus the 8-bit sub-scale rounding
    assert np.all(err <= step * 0.5 + np.abs(g).max(-1, keepdims=True) * 0.03)


# ---------------------------------------------------------------- generator
def test_synth_normal_moments_and_determinism():
    a = ora.synth_normal(7, 123, 200000)
    b = ora.synth_normal(7, 123, 200000)
    np.testing.assert_array_equal(a, b)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    assert np.abs(a).max() <= 6.0
    c = ora.synth_normal(7, 124, 1000)
    assert not np.array_equal(a[:1000], c)
    # Irwin-Hall values are k / 65536 exactly
    assert np.all(a[:1000] * 65536 == np.round(a[:1000] * 65536))


# ------------------------------------------------ GGML 32-weight blocks
def q8_0_block(d: float, q) -> bytes:
    return np.float16(d).tobytes() + np.asarray(q, np.int8).tobytes()


def q5_0_block(d: float, qh: int, qs) -> bytes:
    return np.float16(d).tobytes() + int(qh).to_bytes(4, "little") + np.asarray(qs, np.uint8).tobytes()


def test_q8_0_known_answers():
    # q = 4j - 64 at d = 1/4 gives j - 16; the extremes at d = 2 give 254 / -256
    b0 = q8_0_block(0.25, [4 * j - 64 for j in range(32)])
    b1 = q8_0_block(2.0, [127, -128] * 16)
    got = ora.q8_0_dequant(np.frombuffer(b0 + b1, np.uint8), 1, 64)
    np.testing.assert_array_equal(got[0, :32], np.arange(32, dtype=np.float32) - 16)
    np.testing.assert_array_equal(got[0, 32:], np.array([254.0, -256.0] * 16, np.float32))


def test_q5_0_known_answers():
    j = np.arange(16)
    # qs byte j holds weight j (low nibble) and weight j + 16 (high nibble);
    # qh bit j / j + 16 is their fifth bit: weights 0..31 become q = 0..31,
    # value q - 16
    b0 = q5_0_block(1.0, 0xFFFF0000, j | (j << 4))
    # fifth bits only on the low half: weights j -> 31 - j, j + 16 -> 0,
    # at d = -1/2
    b1 = q5_0_block(-0.5, 0x0000FFFF, 15 - j)
    got = ora.q5_0_dequant(np.frombuffer(b0 + b1, np.uint8), 1, 64)
    np.testing.assert_array_equal(got[0, :32], np.arange(32, dtype=np.float32) - 16)
    want = np.concatenate([(15 - j).astype(np.float32) * -0.5, np.full(16, 8.0, np.float32)])
    np.testing.assert_array_equal(got[0, 32:], want)
    # rows are consecutive runs of blocks
    two = ora.q5_0_dequant(np.frombuffer(b1 + b0, np.uint8), 2, 32)
    np.testing.assert_array_equal(two[1], got[0, :32])
