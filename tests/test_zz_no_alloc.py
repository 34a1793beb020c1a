"""The allocation-free A8 GEMV (pgd_matrix_gemv_act_dev_noalloc) against the
allocating entry point it mirrors (pgd_matrix_gemv_act_dev): bitwise equal
outputs on two calls in a row, the second with fewer rows, over the kernel
families that use scratch (split-K shared-operand, two-chunk pairs,
stream-K) and the per-wave kernels that do not; a launch beyond the fixed
scratch is refused before anything runs."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _noalloc(m, act, rows, y, ldy, res=0, ldres=0):
    from pagoda_amd._lib import call

    call("pgd_matrix_gemv_act_dev_noalloc", m.handle, C.c_void_p(act), rows, C.c_void_p(y), ldy,
         C.c_void_p(res or None), ldres)


@pytest.mark.parametrize("n_out,n_in,rows", [
    (151936, 5120, (32, 7)),   # stream-K (lm_head shape)
    (12352, 5120, (64, 20)),   # two-chunk shared-operand pair, then split-K shared
    (5120, 17408, (32, 3)),    # split-K shared, then per-wave
    (96, 640, (17, 1)),        # per-wave kernels (no scratch)
])
def test_noalloc_gemv_equals_allocating(dev, n_out, n_in, rows):
    from pagoda_amd import Matrix
    from pagoda_amd.matrix import act_bytes, act_prep_dev

    print(f"noalloc gemv {n_out}x{n_in} rows {rows}", flush=True)
    m = Matrix.synth(dev, 0, n_out, n_in, 3, 7000 + n_out, 0.02)
    rng = np.random.default_rng(n_out)
    for res in (False, True):
        for r in rows:
            x = rng.normal(0, 1, (r, n_in)).astype(np.float32)
            xd = dev.upload(x)
            act = dev.alloc(act_bytes(r, n_in))
            act_prep_dev(dev, xd, n_in, r, n_in, act)
            base = rng.normal(0, 1, (r, n_out)).astype(np.float32)
            y1, y2 = dev.upload(base), dev.upload(base)
            if res:
                m.gemv_act_dev(act, r, y1, n_out, y1, n_out)
                _noalloc(m, act, r, y2, n_out, y2, n_out)
            else:
                m.gemv_act_dev(act, r, y1, n_out)
                _noalloc(m, act, r, y2, n_out)
            a = dev.download(y1, (r, n_out), np.float32)
            b = dev.download(y2, (r, n_out), np.float32)
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
            for p in (xd, act, y1, y2):
                dev.free(p)
    m.free()


def test_noalloc_rejects_launch_beyond_fixed_scratch(dev):
    from pagoda_amd import Matrix, PagodaError
    from pagoda_amd._lib import lib
    from pagoda_amd.matrix import act_bytes, act_prep_dev

    assert lib().pgd_noalloc_scratch_bytes() == 40 << 20
    n_out, n_in, r = 48000, 512, 64  # 4 split ranges x 64 rows x 48000 x 4 B = 49 MB of partial sums
    m = Matrix.synth(dev, 0, n_out, n_in, 3, 9, 0.02)
    xd = dev.upload(np.ones((r, n_in), np.float32))
    act = dev.alloc(act_bytes(r, n_in))
    act_prep_dev(dev, xd, n_in, r, n_in, act)
    sentinel = np.full((r, n_out), 7.0, np.float32)
    y = dev.upload(sentinel)
    with pytest.raises(PagodaError, match="scratch"):
        _noalloc(m, act, r, y, n_out)
    np.testing.assert_array_equal(dev.download(y, (r, n_out), np.float32), sentinel)  # nothing ran
    _noalloc(m, act, 32, y, n_out)  # 32 rows fit
    for p in (xd, act, y):
        dev.free(p)
    m.free()


def test_noalloc_calls_on_two_streams_are_ordered(dev):
    """Two device handles (two HIP streams) take turns on the one fixed
    scratch array without host synchronization: each call waits on the GPU
    for the other stream's previous call, so every output equals the
    allocating entry point's."""
    import os

    from pagoda_amd import Device, Matrix
    from pagoda_amd.matrix import act_bytes, act_prep_dev

    dev2 = Device(os.environ.get("PAGODA_DEVICE", "hip"))
    n_out, n_in, r = 151936, 5120, 32  # stream-K: partial sums in scratch
    ms = [Matrix.synth(d, 0, n_out, n_in, 3, 77, 0.02) for d in (dev, dev2)]
    rng = np.random.default_rng(9)
    acts, ys, refs = [], [], []
    for k in range(4):
        x = rng.normal(0, 1, (r, n_in)).astype(np.float32)
        xd = dev.upload(x)
        act = dev.alloc(act_bytes(r, n_in))
        act_prep_dev(dev, xd, n_in, r, n_in, act)
        dev.sync()
        ref = dev.alloc(r * n_out * 4)
        ms[0].gemv_act_dev(act, r, ref, n_out)
        dev.sync()
        refs.append(dev.download(ref, (r, n_out), np.float32))
        dev.free(ref)
        dev.free(xd)
        acts.append(act)
        ys.append(dev.alloc(r * n_out * 4))
    for k in range(4):  # alternate streams, no host synchronization between calls
        _noalloc(ms[k % 2], acts[k], r, ys[k], n_out)
    dev.sync()
    dev2.sync()
    for k in range(4):
        got = dev.download(ys[k], (r, n_out), np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), refs[k].view(np.uint32), err_msg=str(k))
    for p in acts + ys:
        dev.free(p)
    for m in ms:
        m.free()
    dev2.close()
