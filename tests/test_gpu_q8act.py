"""GGML-format GEMV with candle's CPU arithmetic (pgd_matrix_gemv_q8act_dev):
each activation row quantized to Q8_K (Q4_K / Q6_K) or Q8_0 (Q8_0 / Q5_0) and
integer block dots, against the oracle's restatement of the same kernels
(oracle.c: q8k_quantize_block, vec_dot_q4k_q8k, vec_dot_q6k_q8k,
vec_dot_q8_0_q8_0, vec_dot_q5_0_q8_0). The integer parts are exact and the
f32 terms are added in GGML's scalar order (eight residue-class sums per
256-block, block after block), so every output is bit-equal to the oracle."""
import numpy as np
import pytest

from checkpoints import GGML_Q5_0, GGML_Q8_0, random_blocks
from oracle import pyoracle as ora

pytestmark = pytest.mark.gpu

def close(y, ref):
    """Bit-equal to the oracle's f32 outputs."""
    return bool(np.array_equal(np.asarray(y, np.float32).view(np.uint32), np.asarray(ref, np.float32).view(np.uint32)))


def oracle_rows(fmt, blocks, n_out, n_in, x):
    out = []
    for row in x:
        if fmt in (1, 2):
            out.append(ora.kq_vec_dot_q8k(fmt, blocks, n_out, n_in, ora.q8k_quantize(row)))
        else:
            out.append(ora.q8_0_vec_dot(fmt, blocks, n_out, n_in, ora.q8_0_quantize_act(row)))
    return np.stack(out).astype(np.float32)


def make(dev, fmt, n_out, n_in, seed):
    from pagoda_amd import Matrix

    rng = np.random.default_rng(seed)
    if fmt in (1, 2):
        w = rng.normal(0, 0.02, (n_out, n_in)).astype(np.float32)
        blk = ora.q4k_quantize(w) if fmt == 1 else ora.q6k_quantize(w)
    else:
        blk = random_blocks(rng, GGML_Q8_0 if fmt == 3 else GGML_Q5_0, n_out, n_in, d_std=2e-3)
    return Matrix.upload_kq(dev, fmt, blk, n_out, n_in), blk


SHAPES = [(4864, 896), (896, 4864), (1152, 896), (151936, 896), (40, 320)]


@pytest.mark.parametrize("fmt", [1, 2, 3, 4])
@pytest.mark.parametrize("shape", SHAPES)
def test_q8act_gemv_matches_oracle(dev, fmt, shape):
    n_out, n_in = shape
    if fmt in (3, 4) and n_out == 151936:
        n_out = 8192  # keeps the random 32-weight blocks small
    m, blk = make(dev, fmt, n_out, n_in, 100 * fmt + n_in % 97)
    rng = np.random.default_rng(n_out + fmt)
    x = rng.normal(0, 1, (9, n_in)).astype(np.float32)
    x[3, :] = 0.0  # an all-zero row: d = 0 blocks
    x[4, 5] = 40.0  # one outlier sets its block's scale
    xd = dev.upload(x)
    ref = oracle_rows(fmt, blk, n_out, n_in, x)
    outs = {}
    for rows in (1, 4, 9):
        yd = dev.alloc(rows * n_out * 4)
        m.gemv_q8act_dev(xd, n_in, rows, yd, n_out)
        outs[rows] = dev.download(yd, (rows, n_out), np.float32)
        dev.free(yd)
        assert close(outs[rows], ref[:rows]), (rows, np.abs(outs[rows] - ref[:rows]).max(),
                                                 int((outs[rows] != ref[:rows]).sum()))
    # a row's result does not depend on how many rows share its launch
    np.testing.assert_array_equal(outs[4][0].view(np.uint32), outs[1][0].view(np.uint32))
    np.testing.assert_array_equal(outs[9][:4].view(np.uint32), outs[4].view(np.uint32))
    # residual form
    res = rng.normal(0, 1, (4, n_out)).astype(np.float32)
    rd = dev.upload(res)
    m.gemv_q8act_dev(xd, n_in, 4, rd, n_out, rd, n_out)
    got = dev.download(rd, (4, n_out), np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), (res + outs[4]).view(np.uint32))
    dev.free(rd)
    dev.free(xd)
    m.free()


@pytest.mark.parametrize("fa,fb", [(1, 2), (2, 1), (3, 4)])
def test_q8act_pair_equals_two_launches(dev, fa, fb):
    """Two matrices over one input in one launch (the attention's stacked
    q|k and v): each output bit-equal to its own launch, at 1, 4 and 9 rows
    (1-, 4- and 16-row launches), with a row stride wider than either."""
    n_in, na, nb = 896, 1024, 128
    if fa == 3:
        na = 1000  # a partly filled last tile
    ma, _ = make(dev, fa, na, n_in, 11 * fa)
    mb, _ = make(dev, fb, nb, n_in, 13 * fb)
    rng = np.random.default_rng(fa * 10 + fb)
    x = rng.normal(0, 1, (9, n_in)).astype(np.float32)
    xd = dev.upload(x)
    ld = na + nb + 16
    for rows in (1, 4, 9):
        ys, ya, yb = dev.alloc(rows * ld * 4), dev.alloc(rows * na * 4), dev.alloc(rows * nb * 4)
        ma.gemv_q8act_pair_dev(ys, mb, ys + na * 4, xd, n_in, rows, ld)
        ma.gemv_q8act_dev(xd, n_in, rows, ya, na)
        mb.gemv_q8act_dev(xd, n_in, rows, yb, nb)
        got = dev.download(ys, (rows, ld), np.float32)
        a = dev.download(ya, (rows, na), np.float32)
        b = dev.download(yb, (rows, nb), np.float32)
        np.testing.assert_array_equal(got[:, :na].view(np.uint32), a.view(np.uint32), err_msg=f"a rows={rows}")
        np.testing.assert_array_equal(got[:, na:na + nb].view(np.uint32), b.view(np.uint32), err_msg=f"b rows={rows}")
        for p in (ys, ya, yb):
            dev.free(p)
    dev.free(xd)
    ma.free()
    mb.free()


def test_q8act_pair_rejects_mixed_activation_types(dev):
    from pagoda_amd import PagodaError

    ma, _ = make(dev, 1, 64, 256, 1)
    mb, _ = make(dev, 3, 64, 256, 2)
    xd = dev.upload(np.ones((1, 256), np.float32))
    yd = dev.alloc(128 * 4)
    with pytest.raises(PagodaError):
        ma.gemv_q8act_pair_dev(yd, mb, yd + 256, xd, 256, 1, 128)
    for p in (xd, yd):
        dev.free(p)
    ma.free()
    mb.free()


def test_q8act_rejects_a8(dev):
    from pagoda_amd import Matrix, PagodaError

    m = Matrix.synth(dev, 0, 64, 256, 1, 1, 0.02)
    xd = dev.upload(np.ones((1, 256), np.float32))
    yd = dev.alloc(64 * 4)
    with pytest.raises(PagodaError):
        m.gemv_q8act_dev(xd, 256, 1, yd, 64)
    dev.free(xd)
    dev.free(yd)


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("n_in", [8960, 18944])
def test_q8act_wide_rows_16(dev, fmt, n_in):
    """Down projections of the larger Qwen2 sizes (intermediate 8960: 1.5B,
    18944: 7B): 16 quantized rows of these widths do not fit the LDS at once,
    so the launch takes fewer rows at a time with the same per-row arithmetic."""
    n_out = 256
    m, blk = make(dev, fmt, n_out, n_in, 7 * fmt + n_in % 89)
    x = np.random.default_rng(n_in).normal(0, 1, (16, n_in)).astype(np.float32)
    xd = dev.upload(x)
    yd = dev.alloc(16 * n_out * 4)
    m.gemv_q8act_dev(xd, n_in, 16, yd, n_out)
    y = dev.download(yd, (16, n_out), np.float32)
    assert close(y, oracle_rows(fmt, blk, n_out, n_in, x))
    y1 = dev.alloc(n_out * 4)
    m.gemv_q8act_dev(xd, n_in, 1, y1, n_out)
    np.testing.assert_array_equal(dev.download(y1, (1, n_out), np.float32)[0].view(np.uint32), y[0].view(np.uint32))
    for p in (xd, yd, y1):
        dev.free(p)
    m.free()
