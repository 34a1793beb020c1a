"""GPU parity of the quantized formats and GEMVs, through the C ABI.

Bars: dequantized weights bit-exact to the oracle; GEMV within 1e-3 of an
fp64 dot over the oracle-dequantized weights (max error relative to max
|y|); batched rows bitwise equal to single-row calls, except that the fused
SwiGLU GEMV and matrices of >= 2048 row tiles run 5..32-row launches on the
stream-K kernel (bitwise equal among themselves, within 1e-5 of 1..4-row
launches).
"""
import numpy as np
import pytest

from oracle import pyoracle as ora

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3


def rel_err(y, ref):
    """The larger of max|d| / max|ref| and the elementwise ratio
    max_i |d_i| / (|ref_i| + 0.1 max|ref|): below tol means every output is
    within tol of itself plus an absolute 0.1 * tol * max|ref|."""
    d = np.abs(y.astype(np.float64) - ref)
    scale = max(np.abs(ref).max(), 1e-30)
    return float(max(d.max() / scale, (d / (np.abs(ref) + 0.1 * scale)).max()))


def make(dev, fmt, w):
    from pagoda_amd import Matrix
    from pagoda_amd.matrix import FMT_A8, FMT_Q4K

    n_out, n_in = w.shape
    if fmt == FMT_A8:
        p, s, b = ora.a8_quantize(w)
        return Matrix.upload_a8(dev, p, s, b, n_out, n_in), ora.a8_dequant(p, s, b, n_out, n_in)
    if fmt == FMT_Q4K:
        blk = ora.q4k_quantize(w)
        return Matrix.upload_kq(dev, fmt, blk, n_out, n_in), ora.q4k_dequant(blk, n_out, n_in)
    blk = ora.q6k_quantize(w)
    return Matrix.upload_kq(dev, fmt, blk, n_out, n_in), ora.q6k_dequant(blk, n_out, n_in)


FMTS = [0, 1, 2]
SHAPES = [(64, 256), (37, 896), (130, 4864 // 4), (96, 1152)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("shape", SHAPES)
def test_dequant_bit_exact(dev, fmt, shape):
    n_out, n_in = shape
    if fmt == 0 and n_in % 64:
        pytest.skip("A8 needs n_in % 64 == 0")
    rng = np.random.default_rng(n_out * 7 + n_in + fmt)
    w = rng.normal(0, 0.02, shape).astype(np.float32)
    m, ref = make(dev, fmt, w)
    got = m.dequant()
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    # row window
    np.testing.assert_array_equal(m.dequant(3, 5), ref[3:8])


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("shape", [(64, 256), (300, 896), (129, 1216), (64, 4864)])
def test_synth_on_device_matches_cpu_quantizer(dev, fmt, shape):
    """The device generator reproduces the CPU generator + quantizer bit for
    bit (same seeded weights on both sides of every parity test)."""
    from pagoda_amd import Matrix

    n_out, n_in = shape
    if fmt == 0 and n_in % 64:
        pytest.skip("A8 needs n_in % 64 == 0")
    seed, key = 1234, (5 << 8) | 12
    m = Matrix.synth(dev, fmt, n_out, n_in, seed, key, 0.02)
    w = ora.synth_normal(seed, key, n_out * n_in, 0.02).reshape(n_out, n_in)
    _, ref = make(dev, fmt, w)
    np.testing.assert_array_equal(m.dequant().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("shape", [(64, 256), (333, 896), (77, 4864), (1152, 896)])
@pytest.mark.parametrize("rows", [1, 3, 8, 13, 30])
def test_gemv_matches_fp64(dev, fmt, shape, rows):
    n_out, n_in = shape
    if fmt == 0 and n_in % 64:
        pytest.skip("A8 needs n_in % 64 == 0")
    rng = np.random.default_rng(fmt * 1000 + rows)
    w = rng.normal(0, 0.02, shape).astype(np.float32)
    m, deq = make(dev, fmt, w)
    x = rng.normal(0, 1, (rows, n_in)).astype(np.float32)
    y = m.gemv(x)
    ref = x.astype(np.float64) @ deq.astype(np.float64).T
    assert rel_err(y, ref) < GEMV_TOL


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("n_out", [200, 203])
def test_batched_rows_bitwise_equal_serial(dev, fmt, n_out):
    """qwen3_gemv.rs:1115-1167: a batched step equals per-row GEMVs exactly
    (203 outputs: 17..32-row A8 launches take the per-wave kernel, not the
    shared-operand kernel + vector reduction)."""
    rng = np.random.default_rng(9)
    w = rng.normal(0, 0.02, (n_out, 1024)).astype(np.float32)
    m, _ = make(dev, fmt, w)
    x = rng.normal(0, 1, (32, 1024)).astype(np.float32)
    serial = np.stack([m.gemv(x[i]) for i in range(32)])
    for rows in (2, 4, 8, 13, 21, 32):
        got = m.gemv(x[:rows])
        np.testing.assert_array_equal(got.view(np.uint32), serial[:rows].view(np.uint32))


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("shape", [(4864, 896), (151936, 896)])
def test_kquant_64_rows_one_launch_bitwise(dev, fmt, shape):
    """Q4_K / Q6_K launches of 33..64 rows on tall matrices take four 16-row
    batch tiles at once (the weights stream once): every row bitwise equal to
    its single-row GEMV, the whole against fp64."""
    n_out, n_in = shape
    rng = np.random.default_rng(fmt + n_out)
    from pagoda_amd import Matrix

    m = Matrix.synth(dev, fmt, n_out, n_in, 5, 60 + fmt, 0.02)
    x = rng.normal(0, 1, (64, n_in)).astype(np.float32)
    full = m.gemv(x)
    for r in (0, 17, 40, 63):
        np.testing.assert_array_equal(full[r].view(np.uint32), m.gemv(x[r]).view(np.uint32))
    np.testing.assert_array_equal(m.gemv(x[:45]).view(np.uint32), full[:45].view(np.uint32))
    deq = m.dequant().astype(np.float64)
    assert rel_err(full, x.astype(np.float64) @ deq.T) < GEMV_TOL


def test_reference_gemv_patterns(dev):
    """qwen3_gemv.rs:1038-1112: closed-form A8 GEMVs."""
    from pagoda_amd import Matrix

    n_in = 256
    # code = i % 256, scale .5, bias -1, x = 1  (tol 1e-4)
    codes = (np.arange(n_in) % 256).astype(np.uint8)
    s = np.full(4, ora.f32_to_bf16(0.5), np.uint16)
    b = np.full(4, ora.f32_to_bf16(-1.0), np.uint16)
    m = Matrix.upload_a8(dev, codes.view(np.uint32), s, b, 1, n_in)
    y = m.gemv(np.ones(n_in, np.float32))
    expect = sum(-1.0 + 0.5 * (i % 256) for i in range(n_in))
    assert abs(y[0] - expect) < 1e-4
    # multi-row: code = (r*3+i) % 256, scale .25, bias 1, x = i*0.01 (tol 1e-1)
    n_out = 8
    codes = np.array([[(r * 3 + i) % 256 for i in range(n_in)] for r in range(n_out)], np.uint8)
    s = np.full(n_out * 4, ora.f32_to_bf16(0.25), np.uint16)
    b = np.full(n_out * 4, ora.f32_to_bf16(1.0), np.uint16)
    m = Matrix.upload_a8(dev, codes.reshape(-1).view(np.uint32), s, b, n_out, n_in)
    x = (np.arange(n_in) * 0.01).astype(np.float32)
    y = m.gemv(x)
    for r in range(n_out):
        e = sum((1.0 + 0.25 * ((r * 3 + i) % 256)) * x[i] for i in range(n_in))
        assert abs(y[r] - e) < 1e-1


def test_shared_x_two_matrices_and_residual(dev):
    """qwen3_gemv.rs:1061-1085 and 1964-2055: same x through two matrices,
    SwiGLU epilogue and residual epilogue."""
    from pagoda_amd import Matrix

    n_out, n_in = 128, 256
    a_pk = np.full(n_out * n_in // 4, 0x01020304, np.uint32)
    b_pk = np.full(n_out * n_in // 4, 0x04030201, np.uint32)
    s = np.full(n_out * 4, ora.f32_to_bf16(0.01), np.uint16)
    bb = np.full(n_out * 4, ora.f32_to_bf16(0.1), np.uint16)
    A = Matrix.upload_a8(dev, a_pk, s, bb, n_out, n_in)
    B = Matrix.upload_a8(dev, b_pk, s, bb, n_out, n_in)
    x = np.full(n_in, 0.5, np.float32)
    ya, yb = A.gemv(x), B.gemv(x)
    deq_a = ora.a8_dequant(a_pk, s, bb, n_out, n_in)
    np.testing.assert_allclose(ya, deq_a.astype(np.float64) @ x, atol=1e-4)
    # device-side swiglu and residual
    xd = dev.upload(np.pad(x, (0, 0)))
    mid = dev.alloc(n_out * 4)
    Matrix.gemv_swiglu_dev(A, B, xd, n_in, 1, mid, n_out)
    got = dev.download(mid, (n_out,), np.float32)
    np.testing.assert_allclose(got, ya / (1 + np.exp(-ya)) * yb, rtol=1e-5, atol=1e-5)
    res = np.arange(n_out, dtype=np.float32)
    rd = dev.upload(res)
    A.gemv_dev(xd, n_in, 1, rd, n_out, res_ptr=rd, ldres=n_out)  # aliasing residual
    got = dev.download(rd, (n_out,), np.float32)
    np.testing.assert_allclose(got, res + ya, rtol=1e-6, atol=1e-5)
    for p in (xd, mid, rd):
        dev.free(p)


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("shape", [(4864, 896), (896, 4864), (1152, 896), (151936, 896)])
@pytest.mark.parametrize("rows", [1, 4, 8, 16, 32, 64])
def test_config2_sweep_f16_activations(dev, fmt, shape, rows):
    """Config 2: Q4K/Q6K, x fp16 N(0,1), ragged rows, vs CPU-dequant fp32 GEMV
    (evaluated in fp64). shape is (N, K)."""
    from pagoda_amd import Matrix

    n_out, n_in = shape
    seed = 77
    m = Matrix.synth(dev, fmt, n_out, n_in, seed, fmt, 0.02)
    deq = m.dequant()
    rng = np.random.default_rng(rows)
    x16 = rng.normal(0, 1, (rows, n_in)).astype(np.float16)
    xd = dev.upload(x16)
    yd = dev.alloc(rows * n_out * 4)
    m.gemv_dev(xd, n_in, rows, yd, n_out, x_f16=True)
    y = dev.download(yd, (rows, n_out), np.float32)
    ref = x16.astype(np.float64) @ deq.astype(np.float64).T
    assert rel_err(y, ref) < GEMV_TOL
    dev.free(xd)
    dev.free(yd)


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("x_f16", [True, False])
def test_kquant_tall_matrix_staged_activations(dev, fmt, x_f16):
    """Tall Q4_K/Q6_K matrices (>= 1024 row tiles, K = 896: one wave per tile)
    stage the launch's activation rows in LDS once per workgroup. Checked
    against fp64 at 1, 17 and 64 rows, and each batched row bitwise against
    its one-row GEMV."""
    from pagoda_amd import Matrix

    n_out, n_in = 33000, 896
    m = Matrix.synth(dev, fmt, n_out, n_in, 91, fmt + 40, 0.02)
    deq = m.dequant().astype(np.float64)
    rng = np.random.default_rng(fmt * 2 + int(x_f16))
    x = rng.normal(0, 1, (64, n_in)).astype(np.float16 if x_f16 else np.float32)
    xd = dev.upload(x)
    yd = dev.alloc(64 * n_out * 4)
    outs = {}
    for rows in (1, 17, 64):
        m.gemv_dev(xd, n_in, rows, yd, n_out, x_f16=x_f16)
        outs[rows] = dev.download(yd, (rows, n_out), np.float32)
        ref = x[:rows].astype(np.float64) @ deq.T
        assert rel_err(outs[rows], ref) < GEMV_TOL
    np.testing.assert_array_equal(outs[17][0].view(np.uint32), outs[1][0].view(np.uint32))
    np.testing.assert_array_equal(outs[64][:17].view(np.uint32), outs[17].view(np.uint32))
    dev.free(xd)
    dev.free(yd)


def test_prepared_activations_shared_across_matrices(dev):
    """One activation prep feeds several A8 matrices (qwen3_gemv.rs:149-253
    gemv_shared); results are bitwise those of the unprepared calls."""
    from pagoda_amd import Matrix
    from pagoda_amd.matrix import act_bytes, act_prep_dev

    rng = np.random.default_rng(12)
    K = 640
    mats = [Matrix.synth(dev, 0, n, K, 9, 100 + n, 0.02) for n in (96, 33, 512)]
    for rows in (1, 5, 17, 40):
        x = rng.normal(0, 1, (rows, K)).astype(np.float32)
        xd = dev.upload(x)
        act = dev.alloc(act_bytes(rows, K))
        act_prep_dev(dev, xd, K, rows, K, act)
        for m in mats:
            y1 = dev.alloc(rows * m.n_out * 4)
            y2 = dev.alloc(rows * m.n_out * 4)
            m.gemv_dev(xd, K, rows, y1, m.n_out)
            m.gemv_act_dev(act, rows, y2, m.n_out)
            a = dev.download(y1, (rows, m.n_out), np.float32)
            b = dev.download(y2, (rows, m.n_out), np.float32)
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
            ref = x.astype(np.float64) @ m.dequant().astype(np.float64).T
            assert rel_err(b, ref) < GEMV_TOL
            dev.free(y1)
            dev.free(y2)
        dev.free(xd)
        dev.free(act)


@pytest.mark.parametrize("n_out", [8200, 8192 + 64])
@pytest.mark.parametrize("rows", [9, 19, 32, 45, 64])
def test_a8_two_tile_waves_large_matrix(dev, n_out, rows):
    """Matrices of 256+ row tiles run two tiles per wave when a launch holds
    17-32 rows; an odd tile count leaves the last wave with one real tile.
    Checked against fp64 and the batched == serial bitwise bar (the serial
    calls take the one-row staging)."""
    from pagoda_amd import Matrix

    K = 512
    m = Matrix.synth(dev, 0, n_out, K, 31, 7, 0.02)
    deq = m.dequant()
    rng = np.random.default_rng(n_out)
    x = rng.normal(0, 1, (rows, K)).astype(np.float32)
    y = m.gemv(x)
    ref = x.astype(np.float64) @ deq.astype(np.float64).T
    assert rel_err(y, ref) < GEMV_TOL
    for i in (0, 7, rows - 1):
        np.testing.assert_array_equal(m.gemv(x[i]).view(np.uint32), y[i].view(np.uint32))


@pytest.mark.parametrize("rows", [6, 16, 29, 40, 64])
def test_a8_wide_matrix_shared_stage(dev, rows):
    """A narrow matrix with K >= 16384 (256+ groups) runs 5..32-row launches
    through the shared-operand kernel + range reduction, and 37..64 rows as
    one launch over two activation chunks; every row is bitwise its one-row
    GEMV."""
    from pagoda_amd import Matrix

    n_out, K = 300, 16384
    m = Matrix.synth(dev, 0, n_out, K, 41, 9, 0.02)
    deq = m.dequant()
    rng = np.random.default_rng(rows)
    x = rng.normal(0, 1, (rows, K)).astype(np.float32)
    y = m.gemv(x)
    ref = x.astype(np.float64) @ deq.astype(np.float64).T
    assert rel_err(y, ref) < GEMV_TOL
    for i in (0, rows // 2, rows - 1):
        np.testing.assert_array_equal(m.gemv(x[i]).view(np.uint32), y[i].view(np.uint32))


@pytest.mark.parametrize("rows", [40, 64])
def test_a8_pair_launch_residual(dev, rows):
    """The residual epilogue of a two-chunk launch (in place, y = res):
    equals residual + the plain GEMV bit for bit."""
    from pagoda_amd import Matrix
    from pagoda_amd.matrix import act_bytes, act_prep_dev

    n_out, K = 8256, 512
    m = Matrix.synth(dev, 0, n_out, K, 43, 11, 0.02)
    rng = np.random.default_rng(100 + rows)
    x = rng.normal(0, 1, (rows, K)).astype(np.float32)
    res = rng.normal(0, 1, (rows, n_out)).astype(np.float32)
    xd = dev.upload(x)
    act = dev.alloc(act_bytes(rows, K))
    act_prep_dev(dev, xd, K, rows, K, act)
    yd = dev.alloc(rows * n_out * 4)
    m.gemv_act_dev(act, rows, yd, n_out)
    plain = dev.download(yd, (rows, n_out), np.float32)
    rd = dev.upload(res)
    m.gemv_act_dev(act, rows, rd, n_out, rd, n_out)
    got = dev.download(rd, (rows, n_out), np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), (res + plain).view(np.uint32))
    for p in (xd, act, yd, rd):
        dev.free(p)


def _class_checks(full, sub7, sub13, single, ref, sub45=None):
    """Stream-K launches (5..32 rows, and 37..64 rows as two chunks in one
    launch) compute every row alike: a row's output is bitwise the same in any
    such launch; 1..4-row launches use the split-K kernel and agree to fp32
    rounding."""
    assert rel_err(full, ref) < GEMV_TOL
    np.testing.assert_array_equal(sub7.view(np.uint32), full[:7].view(np.uint32))
    np.testing.assert_array_equal(sub13.view(np.uint32), full[32:45].view(np.uint32))
    if sub45 is not None:
        np.testing.assert_array_equal(sub45.view(np.uint32), full[:45].view(np.uint32))
    scale = np.abs(full[3]).max()
    assert np.abs(single.astype(np.float64) - full[3]).max() <= 1e-5 * scale


@pytest.mark.parametrize("n_out,n_in", [(65536 + 40, 128), (66000, 320)])
def test_a8_stream_k_tall_matrix(dev, n_out, n_in):
    """Matrices of >= 2048 row tiles (lm_head) take the stream-K kernel for
    5..32-row launches (two tiles per wave, partial runs added by the fix-up
    kernel); a 64-row call (and a 45-row one) is one launch of two 32-row
    activation chunks."""
    from pagoda_amd import Matrix

    m = Matrix.synth(dev, 0, n_out, n_in, 5, 3, 0.02)
    deq = m.dequant().astype(np.float64)
    rng = np.random.default_rng(n_out)
    x = rng.normal(0, 1, (64, n_in)).astype(np.float32)
    full = m.gemv(x)
    ref = x.astype(np.float64) @ deq.T
    _class_checks(full, m.gemv(x[:7]), m.gemv(x[32:45]), m.gemv(x[3]), ref, m.gemv(x[:45]))


@pytest.mark.parametrize("n_out,n_in", [(1000, 512), (2000, 5120), (4128, 64), (17408, 5120)])
def test_a8_stream_k_swiglu(dev, n_out, n_in):
    """The fused gate/up SwiGLU GEMV takes the stream-K kernel for 5..32 rows:
    silu(x Wg^T) * (x Wu^T) against fp64 over the dequantized weights; ragged
    last tile (n_out % 32 != 0), blocks cut into many runs (K = 5120),
    one-group rows (K = 64: every block whole in one run), the config-4
    shape; 64 and 45 rows run as one launch of two 32-row activation chunks.
    Every launch is repeated and must give the same bits."""
    from pagoda_amd import Matrix

    g = Matrix.synth(dev, 0, n_out, n_in, 11, 1, 0.02)
    u = Matrix.synth(dev, 0, n_out, n_in, 11, 2, 0.02)
    dg, du = g.dequant().astype(np.float64), u.dequant().astype(np.float64)
    rng = np.random.default_rng(n_out + n_in)
    x = rng.normal(0, 1, (64, n_in)).astype(np.float32)

    def run(xs):
        rows = xs.shape[0]
        xd = dev.upload(np.ascontiguousarray(xs))
        md = dev.alloc(rows * n_out * 4)
        Matrix.gemv_swiglu_dev(g, u, xd, n_in, rows, md, n_out)
        out = dev.download(md, (rows, n_out), np.float32)
        Matrix.gemv_swiglu_dev(g, u, xd, n_in, rows, md, n_out)
        again = dev.download(md, (rows, n_out), np.float32)
        np.testing.assert_array_equal(again.view(np.uint32), out.view(np.uint32))
        dev.free(xd)
        dev.free(md)
        return out

    full = run(x)
    x64 = x.astype(np.float64)
    a, b = x64 @ dg.T, x64 @ du.T
    ref = a / (1.0 + np.exp(-a)) * b
    _class_checks(full, run(x[:7]), run(x[32:45]), run(x[3:4])[0], ref, run(x[:45]))


@pytest.mark.parametrize("rows", [256, 300, 390, 516])
@pytest.mark.parametrize("epi", ["store", "res", "swiglu"])
def test_a8_prefill_gemm(dev, rows, epi):
    """Batches of >= 256 rows take the A8 GEMM for their whole 128-row blocks
    (weights read once per 128 rows) and the GEMV kernels for the rest (44
    rows at 300, a 6-row partial chunk at 390, a compact 4-row chunk at 516):
    against fp64 on the same dequantized weights, elementwise, for the store,
    in-place residual and SwiGLU epilogues; n_out 1000 leaves a partial
    weight tile."""
    from pagoda_amd import Matrix
    from pagoda_amd.matrix import act_bytes, act_prep_dev

    n_out, K = 1000, 640
    m = Matrix.synth(dev, 0, n_out, K, 61, 3, 0.02)
    u = Matrix.synth(dev, 0, n_out, K, 62, 4, 0.02) if epi == "swiglu" else None
    rng = np.random.default_rng(rows)
    x = rng.normal(0, 1, (rows, K)).astype(np.float32)
    xd = dev.upload(x)
    act = dev.alloc(act_bytes(rows, K))
    act_prep_dev(dev, xd, K, rows, K, act)
    res = rng.normal(0, 1, (rows, n_out)).astype(np.float32)
    yd = dev.upload(res)
    x64 = x.astype(np.float64)
    if epi == "swiglu":
        Matrix.gemv_swiglu_act_dev(m, u, act, rows, yd, n_out)
        g = x64 @ m.dequant().astype(np.float64).T
        up = x64 @ u.dequant().astype(np.float64).T
        ref = g / (1.0 + np.exp(-g)) * up
    elif epi == "res":
        m.gemv_act_dev(act, rows, yd, n_out, yd, n_out)
        ref = res.astype(np.float64) + x64 @ m.dequant().astype(np.float64).T
    else:
        m.gemv_act_dev(act, rows, yd, n_out)
        ref = x64 @ m.dequant().astype(np.float64).T
    got = dev.download(yd, (rows, n_out), np.float32)
    assert rel_err(got, ref) < GEMV_TOL, rel_err(got, ref)
    for p in (xd, act, yd):
        dev.free(p)



@pytest.mark.parametrize("n_out,n_in,rows,dual", [(17408, 5120, 32, True), (17408, 5120, 64, True),
                                                   (17408, 5120, 9, True), (151936, 5120, 32, False)])
def test_a8_stream_k_repeatable(dev, n_out, n_in, rows, dual):
    """Stream-K launches leave the cut blocks' partial sums in scratch for the
    fix-up launch: 12 launches back to back over the same operands must all
    give the same bits (a piece read before it was stored, or one left over
    from the previous launch, shows up as a launch that differs)."""
    from pagoda_amd import Matrix
    from pagoda_amd.matrix import act_bytes, act_prep_dev

    print(f"stream-K repeat {n_out}x{n_in} rows {rows} dual {dual}", flush=True)
    g = Matrix.synth(dev, 0, n_out, n_in, 21, 1, 0.02)
    u = Matrix.synth(dev, 0, n_out, n_in, 21, 2, 0.02) if dual else None
    x = np.random.default_rng(rows).normal(0, 1, (rows, n_in)).astype(np.float32)
    xd = dev.upload(x)
    act = dev.alloc(act_bytes(rows, n_in))
    act_prep_dev(dev, xd, n_in, rows, n_in, act)
    outs = []
    yd = dev.alloc(rows * n_out * 4)
    for _ in range(12):
        if dual:
            Matrix.gemv_swiglu_act_dev(g, u, act, rows, yd, n_out)
        else:
            g.gemv_act_dev(act, rows, yd, n_out)
        outs.append(dev.download(yd, (rows, n_out), np.float32))
    for o in outs[1:]:
        np.testing.assert_array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    assert np.isfinite(outs[0]).all()
    for p in (xd, act, yd):
        dev.free(p)
    g.free()
    if u is not None:
        u.free()
