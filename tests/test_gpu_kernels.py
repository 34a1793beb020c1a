"""GPU parity of the decode-step kernels against the oracle: the Gated-DeltaNet
recurrence at config-3 shapes and paged GQA decode
attention over ragged slot lists."""
import numpy as np
import pytest

from oracle import pyoracle as ora

pytestmark = pytest.mark.gpu

TOL = 1e-3  # see rel()


def rel(a, b):
    """The larger of max|d| / max|b| and the elementwise ratio
    max_i |d_i| / (|b_i| + 0.1 max|b|): below TOL means every output is
    within TOL of itself plus an absolute 0.1 * TOL * max|b|."""
    d = np.abs(a.astype(np.float64) - b)
    scale = max(np.abs(b).max(), 1e-30)
    return float(max(d.max() / scale, (d / (np.abs(b) + 0.1 * scale)).max()))


def gdn_inputs(rng, rows, kh=16, vh=32, d=128):
    """Config 3: q/k N(0,1) (normalized inside the step), alpha = exp(-softplus(a)·A)
    with A = exp(A_log) ~ U(1,16), beta = sigmoid(b), a, b ~ N(0,1)."""
    conv = rng.normal(0, 1, (rows, 2 * kh * d + vh * d)).astype(np.float32)
    a = rng.normal(0, 1, (rows, vh)).astype(np.float32)
    b = rng.normal(0, 1, (rows, vh)).astype(np.float32)
    z = rng.normal(0, 1, (rows, vh * d)).astype(np.float32)
    a_log = np.log(rng.uniform(1, 16, vh)).astype(np.float32)
    dtb = np.zeros(vh, np.float32)
    norm = rng.uniform(0.5, 1.5, d).astype(np.float32)
    return conv, a, b, z, a_log, dtb, norm


def run_gdn(dev, counts, inputs, states, kh=16, vh=32, prefill=False):
    from pagoda_amd._lib import call
    import ctypes as C

    conv, a, b, z, a_log, dtb, norm = inputs
    nseq = len(counts)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int32)
    rows = int(np.sum(counts))
    d_in = [dev.upload(v) for v in (conv, a, b, z, a_log, dtb, norm)]
    sbuf = dev.upload(states)
    per = states[0].nbytes
    ptrs = np.array([sbuf + i * per for i in range(nseq)], np.uint64)
    d_ptrs = dev.upload(ptrs)
    d_rs = dev.upload(starts)
    d_rc = dev.upload(np.asarray(counts, np.int32))
    d_out = dev.alloc(rows * vh * 128 * 4)
    args = [dev.handle, kh, vh, *[C.c_void_p(p) for p in d_in], C.c_void_p(d_ptrs), C.c_void_p(d_rs),
            C.c_void_p(d_rc), nseq]
    if prefill:
        call("pgd_gdn_prefill_dev", *args, rows, int(max(counts)), C.c_void_p(d_out))
    else:
        call("pgd_gdn_step_dev", *args, C.c_void_p(d_out))
    out = dev.download(d_out, (rows, vh * 128), np.float32)
    new_states = dev.download(sbuf, states.shape, np.float32)
    for p in d_in + [sbuf, d_ptrs, d_rs, d_rc, d_out]:
        dev.free(p)
    return out, new_states


@pytest.mark.parametrize("B", [1, 8, 32, 64])
def test_gdn_decode_step_config3(dev, B):
    rng = np.random.default_rng(B)
    counts = [1] * B
    inputs = gdn_inputs(rng, B)
    states = (rng.normal(0, 1, (B, 32, 128, 128)) * 0.1).astype(np.float32)
    out, new_states = run_gdn(dev, counts, inputs, states)
    conv, a, b, z, a_log, dtb, norm = inputs
    for s in range(B):
        st = states[s].copy()
        ref = ora.gdn_step(conv[s:s + 1], a[s:s + 1], b[s:s + 1], z[s:s + 1], a_log, dtb, norm, 16, 32, 128, 128, st)
        assert rel(out[s:s + 1], ref) < TOL, s
        assert rel(new_states[s], st) < TOL, s


@pytest.mark.parametrize("B", [1, 8, 32, 64])
def test_gdn_4token_chunk_matches_sequential(dev, B):
    """4-token verify chunk == the CPU sequential recurrence, and == four
    single-token GPU steps bitwise (the state round trip through memory is
    exact)."""
    rng = np.random.default_rng(100 + B)
    counts = [4] * B
    inputs = gdn_inputs(rng, 4 * B)
    states = (rng.normal(0, 1, (B, 32, 128, 128)) * 0.1).astype(np.float32)
    out, new_states = run_gdn(dev, counts, inputs, states)
    conv, a, b, z, a_log, dtb, norm = inputs
    for s in range(B):
        st = states[s].copy()
        sl = slice(4 * s, 4 * s + 4)
        ref = ora.gdn_step(conv[sl], a[sl], b[sl], z[sl], a_log, dtb, norm, 16, 32, 128, 128, st)
        assert rel(out[sl], ref) < TOL
        assert rel(new_states[s], st) < TOL
    # same sequence stepped one row at a time on the GPU
    st = states[:1].copy()
    outs = []
    for t in range(4):
        one = tuple(v[t:t + 1] if v.ndim == 2 else v for v in inputs)
        o, st = run_gdn(dev, [1], one, st)
        outs.append(o)
    np.testing.assert_array_equal(np.concatenate(outs).view(np.uint32), out[:4].view(np.uint32))
    np.testing.assert_array_equal(st[0].view(np.uint32), new_states[0].view(np.uint32))


def test_gdn_ragged_mix(dev):
    rng = np.random.default_rng(7)
    counts = [1, 4, 2, 1, 3, 4, 1]
    inputs = gdn_inputs(rng, sum(counts))
    states = (rng.normal(0, 1, (len(counts), 32, 128, 128)) * 0.1).astype(np.float32)
    out, new_states = run_gdn(dev, counts, inputs, states)
    conv, a, b, z, a_log, dtb, norm = inputs
    r = 0
    for s, n in enumerate(counts):
        st = states[s].copy()
        sl = slice(r, r + n)
        ref = ora.gdn_step(conv[sl], a[sl], b[sl], z[sl], a_log, dtb, norm, 16, 32, 128, 128, st)
        assert rel(out[sl], ref) < TOL and rel(new_states[s], st) < TOL
        r += n


def test_gdn_prefill_chunkwise(dev):
    """The prefill entry point over a ragged batch whose long sequences (at
    least 32 rows: whole chunks, a ragged last chunk, exactly one chunk) take
    the chunkwise form and whose short ones take the per-token kernel, from
    nonzero states, against the oracle's per-token recurrence. The chunkwise
    sums round differently from the per-token ones, so the bar is TOL as for
    the step kernel, on the outputs and on the final states."""
    rng = np.random.default_rng(31)
    counts = [300, 7, 33, 32, 31, 64, 1]
    inputs = gdn_inputs(rng, sum(counts))
    states = (rng.normal(0, 1, (len(counts), 32, 128, 128)) * 0.1).astype(np.float32)
    out, new_states = run_gdn(dev, counts, inputs, states, prefill=True)
    out_step, states_step = run_gdn(dev, counts, inputs, states)
    conv, a, b, z, a_log, dtb, norm = inputs
    r = 0
    for s, n in enumerate(counts):
        st = states[s].copy()
        sl = slice(r, r + n)
        ref = ora.gdn_step(conv[sl], a[sl], b[sl], z[sl], a_log, dtb, norm, 16, 32, 128, 128, st)
        assert rel(out[sl], ref) < TOL, n
        assert rel(new_states[s], st) < TOL, n
        if n < 32:  # short sequences run the per-token kernel either way
            np.testing.assert_array_equal(out[sl].view(np.uint32), out_step[sl].view(np.uint32))
            np.testing.assert_array_equal(new_states[s].view(np.uint32), states_step[s].view(np.uint32))
        r += n


def test_gdn_prefill_slow_decay_long(dev):
    """Decay close to 1 (A_log = -8, so a chunk barely forgets) over 200 rows:
    the chunkwise products carry the whole chunk's state instead of rounding
    away old terms."""
    rng = np.random.default_rng(32)
    counts = [200]
    conv, a, b, z, a_log, dtb, norm = gdn_inputs(rng, 200)
    a_log = np.full_like(a_log, -8.0)
    inputs = (conv, a, b, z, a_log, dtb, norm)
    states = (rng.normal(0, 1, (1, 32, 128, 128)) * 0.1).astype(np.float32)
    out, new_states = run_gdn(dev, counts, inputs, states, prefill=True)
    st = states[0].copy()
    ref = ora.gdn_step(conv, a, b, z, a_log, dtb, norm, 16, 32, 128, 128, st)
    assert rel(out, ref) < TOL
    assert rel(new_states[0], st) < TOL


@pytest.mark.parametrize("poison", [False, True])
@pytest.mark.parametrize("heads,kvh,hd", [(24, 4, 256), (14, 2, 64), (8, 8, 128)])
def test_paged_attention_ragged(dev, heads, kvh, hd, poison):
    """Ragged rows over scattered pages. poison: every slot past a sequence's
    last visible position, and every unused page, holds NaN (a pool reusing
    freed memory holds any bit pattern there); results must not change."""
    from pagoda_amd._lib import call
    import ctypes as C

    rng = np.random.default_rng(heads + hd)
    block = 16
    lens = [1, 5, 16, 17, 100, 300]
    nblk = [(n + block - 1) // block for n in lens]
    total_pages = sum(nblk) + 7
    perm = rng.permutation(total_pages)  # scattered pages
    tables = []
    at = 0
    for nb in nblk:
        tables.append(list(perm[at:at + nb]))
        at += nb
    max_blocks = max(nblk)
    bt = np.zeros((len(lens), max_blocks), np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    kpool = rng.normal(0, 1, (total_pages, kvh, block, hd)).astype(np.float32)
    vpool = rng.normal(0, 1, (total_pages, kvh, block, hd)).astype(np.float32)
    # one query row per sequence at its last position, plus one mid-sequence row
    seq_of_row = list(range(len(lens))) + [5]
    pos_of_row = [n - 1 for n in lens] + [150]
    if poison:
        used = set()
        for sq, t in enumerate(tables):
            used.update(t)
            for p in range(lens[sq], len(t) * block):
                kpool[t[p // block], :, p % block] = np.nan
                vpool[t[p // block], :, p % block] = np.nan
        for pg in set(range(total_pages)) - used:
            kpool[pg] = np.nan
            vpool[pg] = np.nan
    rows = len(seq_of_row)
    q = rng.normal(0, 1, (rows, heads, hd)).astype(np.float32)
    gate = rng.normal(0, 1, (rows, heads, hd)).astype(np.float32)
    bufs = [dev.upload(v) for v in (q, gate, kpool, vpool, np.asarray(seq_of_row, np.int32),
                                    np.asarray(pos_of_row, np.int32), bt)]
    d_out = dev.alloc(rows * heads * hd * 4)
    call("pgd_attn_decode_dev", dev.handle, heads, kvh, hd, block, *[C.c_void_p(p) for p in bufs], max_blocks, rows,
         C.c_void_p(d_out))
    out = dev.download(d_out, (rows, heads, hd), np.float32)
    for r in range(rows):
        s, L = seq_of_row[r], pos_of_row[r] + 1
        kc = np.zeros((L, kvh, hd), np.float32)
        vc = np.zeros((L, kvh, hd), np.float32)
        for p in range(L):
            kc[p] = kpool[tables[s][p // block], :, p % block]
            vc[p] = vpool[tables[s][p // block], :, p % block]
        ref = ora.attn_decode(q[r], kc, vc, L, heads, kvh, hd, gate[r])
        assert rel(out[r], ref) < TOL, (r, rel(out[r], ref))
    for p in bufs + [d_out]:
        dev.free(p)


@pytest.mark.parametrize("heads,kvh,hd", [(24, 4, 256), (14, 2, 64)])
def test_paged_attention_shared_trunk(dev, heads, kvh, hd):
    """Forked sequences over one shared trunk (the block tables hold the same
    page ids, as after Session::fork / the radix cache) plus private suffix
    pages, with 4-token verify rows: rows sharing a chunk's pages share one
    work item (more rows than one item holds), and every row equals the
    oracle and, bitwise, the same row attended alone."""
    from pagoda_amd._lib import call
    import ctypes as C

    rng = np.random.default_rng(hd + 3)
    block, trunk = 16, 40  # 640 trunk positions: chunks 0, 1 and part of 2
    nseq = 13
    total_pages = trunk + nseq * 3 + 5
    kpool = rng.normal(0, 1, (total_pages, kvh, block, hd)).astype(np.float32)
    vpool = rng.normal(0, 1, (total_pages, kvh, block, hd)).astype(np.float32)
    free = list(rng.permutation(np.arange(trunk, total_pages)))
    trunk_pages = list(rng.permutation(trunk))
    tables, seq_of_row, pos_of_row = [], [], []
    for i in range(nseq):
        extra = 1 + i % 3  # private pages after the trunk
        tables.append(trunk_pages + [int(free.pop()) for _ in range(extra)])
        last = trunk * block + extra * block - 1 - (i % 7)
        # a decode row, or a 4-token verify chunk for every third sequence
        for t in (range(4) if i % 3 == 0 else range(1)):
            seq_of_row.append(i)
            pos_of_row.append(last - 3 + t if i % 3 == 0 else last)
    seq_of_row.append(2)  # a row inside the trunk
    pos_of_row.append(300)
    rows = len(seq_of_row)
    max_blocks = max(len(t) for t in tables)
    bt = np.zeros((nseq, max_blocks), np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    q = rng.normal(0, 1, (rows, heads, hd)).astype(np.float32)
    gate = rng.normal(0, 1, (rows, heads, hd)).astype(np.float32)
    pools = [dev.upload(kpool), dev.upload(vpool), dev.upload(bt)]

    def run(rsel):
        qs, gs = np.ascontiguousarray(q[rsel]), np.ascontiguousarray(gate[rsel])
        bufs = [dev.upload(qs), dev.upload(gs), pools[0], pools[1],
                dev.upload(np.asarray([seq_of_row[r] for r in rsel], np.int32)),
                dev.upload(np.asarray([pos_of_row[r] for r in rsel], np.int32)), pools[2]]
        d_out = dev.alloc(len(rsel) * heads * hd * 4)
        call("pgd_attn_decode_dev", dev.handle, heads, kvh, hd, block, *[C.c_void_p(p) for p in bufs], max_blocks,
             len(rsel), C.c_void_p(d_out))
        got = dev.download(d_out, (len(rsel), heads, hd), np.float32)
        for p in [bufs[0], bufs[1], bufs[4], bufs[5], d_out]:
            dev.free(p)
        return got

    out = run(list(range(rows)))
    for r in range(rows):
        s, L = seq_of_row[r], pos_of_row[r] + 1
        kc = np.zeros((L, kvh, hd), np.float32)
        vc = np.zeros((L, kvh, hd), np.float32)
        for p in range(L):
            kc[p] = kpool[tables[s][p // block], :, p % block]
            vc[p] = vpool[tables[s][p // block], :, p % block]
        ref = ora.attn_decode(q[r], kc, vc, L, heads, kvh, hd, gate[r])
        assert rel(out[r], ref) < TOL, (r, rel(out[r], ref))
    for r in (0, 5, rows - 1):
        np.testing.assert_array_equal(run([r])[0].view(np.uint32), out[r].view(np.uint32))
    for p in pools:
        dev.free(p)
