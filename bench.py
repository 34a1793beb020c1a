"""Decode throughput of the HIP backend on one MI355X.

Workload: 27B-class hybrid decoder, 64 layers in
a 3:1 Gated-DeltaNet : full-attention pattern, hidden 5120, SwiGLU 17408,
24 q / 4 kv heads of 256, vocab 151936, MLX affine-8 group-64 weights
(random-init, generated on the device), paged KV block 16, random 19-token
prompt, greedy decode. A step is one batched decode step: every sequence of
the batch feeds its previous greedy token and gets its next one.

value = aggregate decode tok/s at batch 32 (the batch-1 rate is reported as
batch1_tok_s). roofline = the dominant kernel of that step (the fused
gate/up SwiGLU A8 GEMV) timed with HIP events on the library's stream,
cycling through 8 gate/up pairs (1.5 GB) so that each launch streams its
weights from HBM as in the decode step, not from the 256 MB last-level
cache; roofline.traffic comes from the committed rocprofv3 counter
measurement of the same kernel (profiles/a8_swiglu_traffic.json).
cpu_baseline = the C oracle (the CPU restatement used as the parity checker)
on a bounded sample: one full-width 4-layer group, extrapolated per token.

--roofline-only runs just the kernel timing (the command the counter runs
profile); --copy-calib runs a plain device copy of known size for scaling
the counters.
"""
from __future__ import annotations

import argparse
import json
from dataclasses import replace
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
# the graph-replayed passes (off with --no-graphs: rocprofv3's kernel tracer
# crashes the host process inside hipGraphLaunch)
USE_GRAPHS = True


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gpu_bench(args):
    from pagoda_amd import Device, Event
    from pagoda_amd.engine import QWEN35_27B, Model

    dev = Device(os.environ.get("PAGODA_DEVICE", "hip"))
    batch = args.batch
    prompt_len = 19
    total = prompt_len + args.warmup + args.steps + 8
    kv_block = QWEN35_27B.kv_block
    cfg = replace(QWEN35_27B, max_pos=max(C5_TRUNK + C5_SUFFIX + C5_GEN + 64, total),
                  kv_blocks=(batch + 2) * ((total + kv_block - 1) // kv_block) + 16 + C5_PAGES)
    # the roofline launches run first, on weights allocated in fresh device
    # memory as the model's are (timed last, after the model and config 1 had
    # allocated and freed ~40 GB, the same 1-row kernel measured 15% slower)
    roof = roofline(dev, cfg, batch)
    t0 = time.time()
    model = Model.synth(dev, cfg, seed=2026)
    info = model.info()
    log(f"model synthesized in {time.time() - t0:.1f}s: {info['weight_bytes'] / 1e9:.2f} GB weights, "
        f"{info['algo_bytes_per_token'] / 1e9:.2f} GB algorithmic weight bytes per step")
    rng = np.random.default_rng(0)
    prompts = [rng.integers(0, cfg.vocab, prompt_len) for _ in range(batch)]

    # ---- batch decode ----
    sessions = [model.new_session() for _ in range(batch)]
    ids, _ = model.step_ragged(sessions, prompts)
    for _ in range(args.warmup):
        ids, _ = model.step_ragged(sessions, [[int(t)] for t in ids])
    dev.sync()
    marks = [Event(dev).record()]
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ids, _ = model.step_ragged(sessions, [[int(t)] for t in ids])
        marks.append(Event(dev).record())
    dev.sync()
    wall = time.perf_counter() - t0
    per_step = np.array([marks[i].elapsed_ms(marks[i + 1]) for i in range(args.steps)])
    gpu_ms = float(per_step.sum())
    ms_per_step = wall * 1e3 / args.steps
    tok_s = batch * args.steps / wall
    pct = {f"p{p}": round(float(np.percentile(per_step, p)), 3) for p in (10, 50, 90)}
    log(f"batch {batch}: {ms_per_step:.2f} ms/step (events {gpu_ms / args.steps:.2f}; {pct}), {tok_s:.1f} tok/s")
    for s in sessions:
        s.free()

    # ---- the same batch decode with each step replayed from a HIP graph ----
    tok_s_graph = None
    if USE_GRAPHS:
        model.set_graphs(True)
        sessions = [model.new_session() for _ in range(batch)]
        ids, _ = model.step_ragged(sessions, prompts)
        for _ in range(args.warmup):
            ids, _ = model.step_ragged(sessions, [[int(t)] for t in ids])
        dev.sync()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            ids, _ = model.step_ragged(sessions, [[int(t)] for t in ids])
        dev.sync()
        tok_s_graph = batch * args.steps / (time.perf_counter() - t0)
        log(f"batch {batch} graphed: {tok_s_graph:.1f} tok/s")
        for s in sessions:
            s.free()
        model.set_graphs(False)

    # ---- batch 1 decode ----
    s = model.new_session()
    s.forward(prompts[0])
    tok = 1
    for _ in range(args.warmup):
        tok, _ = s.forward_greedy(tok)
    dev.sync()
    t0 = time.perf_counter()
    n1 = max(8, args.steps)
    for _ in range(n1):
        tok, _ = s.forward_greedy(tok)
    wall1 = time.perf_counter() - t0
    b1_tok_s = n1 / wall1
    log(f"batch 1: {wall1 * 1e3 / n1:.2f} ms/token, {b1_tok_s:.1f} tok/s")
    s.free()
    b1_graph = None
    if USE_GRAPHS:
        b1_graph = graphed_batch1(model, dev, prompts[0], args.warmup, n1)
        log(f"batch 1 graphed: {b1_graph:.1f} tok/s")
    c5 = None if args.no_config5 else config5(model, cfg)
    model.free()
    c1 = config1(dev)
    return {
        "tok_s": tok_s, "ms_per_step": ms_per_step, "batch1_tok_s": b1_tok_s, "step_ms_pct": pct, "config5": c5,
        "tok_s_graph": tok_s_graph, "batch1_tok_s_graph": b1_graph,
        "config1": c1,
        "weight_gb": info["weight_bytes"] / 1e9, "algo_gb_per_step": info["algo_bytes_per_token"] / 1e9,
        "roofline": roof,
    }


def graphed_batch1(model, dev, prompt, warmup, n):
    """Batch-1 greedy decode with every step replayed from a HIP graph
    (pgd_model_set_graphs); returns tok/s over n timed steps."""
    model.set_graphs(True)
    s = model.new_session()
    s.forward(prompt)
    tok = 1
    for _ in range(warmup + 2):
        tok, _ = s.forward_greedy(tok)
    dev.sync()
    t0 = time.perf_counter()
    for _ in range(n):
        tok, _ = s.forward_greedy(tok)
    rate = n / (time.perf_counter() - t0)
    s.free()
    model.set_graphs(False)
    return rate


def config1(dev):
    """Qwen2.5-0.5B architecture (GGUF Q4_K/Q6_K
    layout, seeded weights), an 81-token random prompt, 32 greedy tokens, then
    the warm rerun: the cold session sliced to its first 80 prompt tokens
    (the prefix graft) is fed the last prompt token plus the 31 tokens it
    generates, 32 fed tokens in all. The greedy rate is also timed over 128
    decode steps."""
    from pagoda_amd.engine import QWEN2_05B, Model

    cfg = QWEN2_05B
    model = Model.synth(dev, cfg, seed=1)
    prompt = np.random.default_rng(81).integers(0, cfg.vocab, 81)
    # one untimed prefill first (first launches of each kernel)
    s = model.new_session()
    model.step_ragged([s], [prompt])
    s.free()
    s = model.new_session()
    dev.sync()
    t0 = time.perf_counter()
    ids, _ = model.step_ragged([s], [prompt])
    tok = int(ids[0])
    dev.sync()
    prefill_ms = (time.perf_counter() - t0) * 1e3
    cold = [tok]
    t0 = time.perf_counter()
    for _ in range(31):
        tok, _ = s.forward_greedy(tok)
        cold.append(tok)
    gen_s = time.perf_counter() - t0
    # the prefix graft of the warm run: the cold session (81 prompt + 31
    # generated positions) sliced to the 80 covered prompt tokens
    # (graft_session -> cache_prefix, pagoda-hf/src/lib.rs:603-616)
    w = s.fork_prefix(80)
    for _ in range(8):
        tok, _ = s.forward_greedy(tok)
    t0 = time.perf_counter()
    n = 128
    for _ in range(n):
        tok, _ = s.forward_greedy(tok)
    dec_s = time.perf_counter() - t0
    s.free()
    dev.sync()
    t0 = time.perf_counter()
    fed = 1
    ids, _ = model.step_ragged([w], [prompt[80:]])
    tok = int(ids[0])
    warm = [tok]
    for _ in range(31):
        tok, _ = w.forward_greedy(tok)
        warm.append(tok)
        fed += 1
    warm_ms = (time.perf_counter() - t0) * 1e3
    w.free()
    # the cold stream again with every decode step replayed from a HIP graph
    gdec, gequal = None, None
    if USE_GRAPHS:
        model.set_graphs(True)
        g = model.new_session()
        ids, _ = model.step_ragged([g], [prompt])
        tok = int(ids[0])
        gcold = [tok]
        for _ in range(31):
            tok, _ = g.forward_greedy(tok)
            gcold.append(tok)
        for _ in range(8):
            tok, _ = g.forward_greedy(tok)
        t0 = time.perf_counter()
        for _ in range(n):
            tok, _ = g.forward_greedy(tok)
        gdec = round(n / (time.perf_counter() - t0), 1)
        gequal = gcold == cold
        g.free()
        model.set_graphs(False)
    # the other arithmetic of GGML matrices: f32 dequant-then-dot (the
    # Metal-like one, matrix-core GEMVs and the paged attention kernel)
    from pagoda_amd.engine import ARITH_DEQUANT_F32

    model.set_kquant_arith(ARITH_DEQUANT_F32)
    f = model.new_session()
    model.step_ragged([f], [prompt])
    tok = 1
    for _ in range(8):
        tok, _ = f.forward_greedy(tok)
    t0 = time.perf_counter()
    for _ in range(n):
        tok, _ = f.forward_greedy(tok)
    fdec = round(n / (time.perf_counter() - t0), 1)
    f.free()
    model.free()
    out = {"prompt": 81, "gen": 32, "prefill_ms": round(prefill_ms, 3), "gen_tok_s": round(31 / gen_s, 1),
           "arith": "cpu_q8 (candle's CPU quantized matmul, bit-equal to the CPU restatement)",
           "decode_tok_s": round(n / dec_s, 1), "decode_tok_s_graph": gdec, "decode_tok_s_dequant_f32": fdec,
           "graph_ids_equal_eager": gequal, "warm_fed_tokens": fed, "warm_ms": round(warm_ms, 2),
           "warm_equals_cold": warm == cold}
    log(f"config 1: prefill {prefill_ms:.2f} ms, decode {out['decode_tok_s']} tok/s "
        f"(graphed {gdec}, ids equal: {gequal}; dequant_f32 arithmetic {fdec}), warm fed {fed}, "
        f"warm == cold: {warm == cold}")
    return out


C5_REQ, C5_TRUNK, C5_SUFFIX, C5_GEN, C5_CHUNK = 64, 3968, 50, 32, 4
C5_PAGES = (C5_TRUNK // 16 + 2) + 2 * C5_REQ * ((C5_SUFFIX + C5_GEN + C5_CHUNK) // 16 + 2)


def config5(model, cfg):
    """64 requests share one random 3968-token trunk
    (prefilled once; its KV pages are shared copy-on-write by every fork),
    each adds its own 50-token suffix and generates 32 greedy tokens.
    Pass A decodes every request one token per step. Pass B restarts from the
    same post-suffix states and packs decode rows (even requests) with 4-token
    known-token verify chunks (odd requests, replaying pass A's tokens) into
    one ragged batch per step; a verify chunk yields 4 tokens in one forward of
    its request. Reports tok/s of both passes, the forwards saved and whether
    every verified token equals pass A's."""
    dev = model.dev
    rng = np.random.default_rng(5)
    trunk = rng.integers(0, cfg.vocab, C5_TRUNK)
    root = model.new_session()
    dev.sync()
    t0 = time.perf_counter()
    root.forward(trunk)
    dev.sync()
    t_trunk = time.perf_counter() - t0
    reqs = [root.fork() for _ in range(C5_REQ)]
    suffixes = [rng.integers(0, cfg.vocab, C5_SUFFIX) for _ in range(C5_REQ)]
    t0 = time.perf_counter()
    first, _ = model.step_ragged(reqs, suffixes)
    dev.sync()
    t_suffix = time.perf_counter() - t0
    snap = [r.fork() for r in reqs]
    # pass A: one decode row per request per step
    streams = [[int(t)] for t in first]
    t0 = time.perf_counter()
    for _ in range(C5_GEN - 1):
        ids, _ = model.step_ragged(reqs, [[s[-1]] for s in streams])
        for s, t in zip(streams, ids):
            s.append(int(t))
    dev.sync()
    t_a = time.perf_counter() - t0
    # pass B: even requests decode, odd requests verify 4 known tokens per forward
    pos = [1] * C5_REQ            # tokens of the stream produced so far (stream[0] came from the suffix)
    fwd = [0] * C5_REQ            # forwards of each request
    bad = 0
    steps = 0
    t0 = time.perf_counter()
    while any(p < C5_GEN for p in pos):
        sess, feeds, owners = [], [], []
        for i in range(C5_REQ):
            if pos[i] >= C5_GEN:
                continue
            n = 1 if i % 2 == 0 else min(C5_CHUNK, C5_GEN - pos[i])
            feeds.append(streams[i][pos[i] - 1:pos[i] - 1 + n])
            sess.append(snap[i])
            owners.append((i, n))
        ids, _ = model.step_ragged(sess, feeds, all_rows=True)
        at = 0
        for i, n in owners:
            got = [int(t) for t in ids[at:at + n]]
            bad += sum(1 for k in range(n) if got[k] != streams[i][pos[i] + k])
            pos[i] += n
            fwd[i] += 1
            at += n
        steps += 1
    dev.sync()
    t_b = time.perf_counter() - t0
    produced = C5_REQ * (C5_GEN - 1)
    saved = produced - sum(fwd)
    for s in reqs + snap + [root]:
        s.free()
    out = {"requests": C5_REQ, "trunk": C5_TRUNK, "suffix": C5_SUFFIX, "gen": C5_GEN,
           "trunk_prefill_s": round(t_trunk, 3), "suffix_prefill_s": round(t_suffix, 3),
           "decode_tok_s": round(produced / t_a, 1), "mixed_tok_s": round(produced / t_b, 1),
           "mixed_steps": steps, "forwards_saved": saved, "verify_mismatches": bad}
    log(f"config 5: {out}")
    return out


PAIRS = 8          # gate/up pairs cycled through (8 x 190 MB)
LAUNCHES = 48      # timed launches per batch size


def roofline(dev, cfg, batch):
    """The fused gate/up SwiGLU A8 GEMV at the decode step's shape, fed
    prepared activations as in the step; only the GEMV launches are timed,
    with events on the library's stream."""
    from pagoda_amd import Event, Matrix
    from pagoda_amd.matrix import act_bytes, act_prep_dev

    H, I = cfg.hidden, cfg.intermediate
    rng = np.random.default_rng(1)
    pairs = [(Matrix.synth(dev, 0, I, H, 2026 + i, (i << 8) | 12), Matrix.synth(dev, 0, I, H, 2026 + i, (i << 8) | 13))
             for i in range(PAIRS)]

    def time_swiglu(rows):
        x = dev.upload(rng.normal(0, 1, (rows, H)).astype(np.float32))
        act = dev.alloc(act_bytes(rows, H))
        mid = dev.alloc(rows * I * 4)
        act_prep_dev(dev, x, H, rows, H, act)
        for g, u in pairs[:2]:
            Matrix.gemv_swiglu_act_dev(g, u, act, rows, mid, I)
        e0 = Event(dev).record()
        for i in range(LAUNCHES):
            g, u = pairs[i % PAIRS]
            Matrix.gemv_swiglu_act_dev(g, u, act, rows, mid, I)
        e1 = Event(dev).record()
        avg_ms = e0.elapsed_ms(e1) / LAUNCHES
        g, u = pairs[0]
        algo = g.algo_bytes + u.algo_bytes + rows * H * 4 + rows * I * 4
        for p in (x, act, mid):
            dev.free(p)
        return avg_ms, algo

    avg_ms, algo = time_swiglu(batch)
    achieved = algo / (avg_ms * 1e-3) / 1e9
    avg1, algo1 = time_swiglu(1)
    log(f"swiglu GEMV kernel {batch} rows: {avg_ms * 1e3:.1f} us, {achieved:.0f} GB/s; 1 row: {avg1 * 1e3:.1f} us, "
        f"{algo1 / (avg1 * 1e-3) / 1e9:.0f} GB/s")
    for g, u in pairs:
        g.free()
        u.free()
    traffic = None
    tfile = ROOT / "profiles" / "a8_swiglu_traffic.json"
    if tfile.exists():
        t = json.loads(tfile.read_text())
        if str(batch) in t.get("hbm_bytes_per_launch", {}):
            traffic = t["hbm_bytes_per_launch"][str(batch)]
    copy = copy_peak(dev)
    mfma = None
    mfile = ROOT / "profiles" / "mfma_busy.json"
    if mfile.exists():
        pd = json.loads(mfile.read_text())["per_dispatch"]
        pick = lambda prefix: next(v["mfma_busy"] for k, v in pd.items() if k.startswith(prefix))
        mfma = {"a8_sk_kernel<2,2,2>": pick("a8_sk_kernel<2,2,2>"), "a8_mma_kernel_1row": pick("a8_mma_kernel"),
                "prefill_a8_gemm_kernel<2>": pick("a8_gemm_kernel<2>"),
                "source": "profiles/mfma_busy.json (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x CUs x 4)"}
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
            "copy_peak": copy["gbs"], "frac_of_copy": achieved / copy["gbs"], "copy_note": copy["note"],
            "mfma_busy": mfma,
            "kernel": (f"fused gate/up SwiGLU A8 GEMV 5120->2x17408, {batch} rows: a8_sk_kernel<2,2,2> (stream-K) "
                       f"+ a8_sk_fix_kernel<2,2> (cut blocks); 1 row: a8_mma_kernel<3,4,1,4,1,2>"),
            "algo_bytes_per_launch": algo, "avg_launch_us": avg_ms * 1e3,
            "batch1": {"achieved": algo1 / (avg1 * 1e-3) / 1e9, "frac": algo1 / (avg1 * 1e-3) / 1e9 / HBM_PEAK_GBS,
                       "avg_launch_us": avg1 * 1e3, "algo_bytes_per_launch": algo1}}


KQ_SHAPES = [(896, 4864), (4864, 896), (896, 1152), (896, 151936)]  # K x N
KQ_ROWS = [1, 4, 8, 16, 32, 64]


def copy_peak(dev):
    """The on-box streaming rate: a plain device-to-device copy of 1 GiB (4x
    the last-level cache) queued on the library's stream, timed with HIP
    events over 10 copies; bytes read + bytes written per second."""
    from pagoda_amd import Event
    from pagoda_amd._lib import call
    import ctypes as C

    n = 1 << 30
    a, b = dev.alloc(n), dev.alloc(n)

    def cp():
        call("pgd_device_copy_dev", dev.handle, C.c_void_p(b), C.c_void_p(a), C.c_size_t(n))

    for _ in range(3):
        cp()
    e0 = Event(dev).record()
    for _ in range(10):
        cp()
    e1 = Event(dev).record()
    gbs = 2 * n * 10 / (e0.elapsed_ms(e1) * 1e-3) / 1e9
    dev.free(a)
    dev.free(b)
    log(f"device copy 1 GiB: {gbs:.0f} GB/s (read + write)")
    return {"gbs": gbs, "note": "device-to-device copy of 1 GiB (hipMemcpyAsync on the library stream), "
                                "(read + write bytes) / time over 10 copies"}


def kernel_sweeps():
    """Config 2 (Q4_K / Q6_K GEMV over K x N shapes and ragged row counts,
    f16 activations) and config 3 (Gated-DeltaNet decode step, B sequences of
    32 value heads with 128 x 128 f32 state, plus 4-token chunks), timed with
    HIP events on the library's stream. Every launch reads weights or state
    that the previous launches did not touch (copies cycled through past the
    last-level cache), so the figures are HBM figures."""
    import ctypes as C
    from pagoda_amd import Device, Event, Matrix
    from pagoda_amd.matrix import FMT_Q4K, FMT_Q6K
    from pagoda_amd._lib import call

    dev = Device(os.environ.get("PAGODA_DEVICE", "hip"))
    rng = np.random.default_rng(3)
    out = {"kquant": [], "gdn": []}
    for fmt, fname in ((FMT_Q4K, "q4k"), (FMT_Q6K, "q6k")):
        for K, N in KQ_SHAPES:
            probe = Matrix.synth(dev, fmt, N, K, 11, 1)
            per = probe.algo_bytes
            ncopy = max(2, int(1.2e9 // probe.dev_bytes) + 1)
            ms = [probe] + [Matrix.synth(dev, fmt, N, K, 11, 2 + i) for i in range(ncopy - 1)]
            for rows in KQ_ROWS:
                x = dev.upload(rng.normal(0, 1, (rows, K)).astype(np.float16))
                y = dev.alloc(rows * N * 4)
                for m in ms[:2]:
                    m.gemv_dev(x, K, rows, y, N, x_f16=True)
                L = max(32, 2 * ncopy)
                e0 = Event(dev).record()
                for i in range(L):
                    ms[i % ncopy].gemv_dev(x, K, rows, y, N, x_f16=True)
                e1 = Event(dev).record()
                us = e0.elapsed_ms(e1) / L * 1e3
                algo = per + rows * K * 2 + rows * N * 4
                gbs = algo / (us * 1e-6) / 1e9
                log(f"{fname} K={K:5d} N={N:6d} rows={rows:2d}: {us:8.2f} us {gbs:7.0f} GB/s {100 * gbs / HBM_PEAK_GBS:5.1f}%")
                out["kquant"].append({"fmt": fname, "K": K, "N": N, "rows": rows, "us": round(us, 3),
                                      "algo_bytes": algo, "gbs": round(gbs, 1),
                                      "frac": round(gbs / HBM_PEAK_GBS, 4)})
                dev.free(x)
                dev.free(y)
            for m in ms:
                m.free()
    # config 3: 16 key heads, 32 value heads, d = 128
    kh, vh, d = 16, 32, 128
    state_bytes = vh * d * d * 4
    for B, toks in ((1, 1), (8, 1), (32, 1), (64, 1), (8, 4), (32, 4)):
        rows = B * toks
        conv = dev.upload(rng.normal(0, 1, (rows, 2 * kh * d + vh * d)).astype(np.float32))
        a = dev.upload(rng.normal(0, 1, (rows, vh)).astype(np.float32))
        b = dev.upload(rng.normal(0, 1, (rows, vh)).astype(np.float32))
        z = dev.upload(rng.normal(0, 1, (rows, vh * d)).astype(np.float32))
        a_log = dev.upload(np.log(rng.uniform(1, 16, vh)).astype(np.float32))
        dtb = dev.upload(np.zeros(vh, np.float32))
        norm = dev.upload(rng.uniform(0.5, 1.5, d).astype(np.float32))
        sets = max(2, int(1.2e9 // (B * state_bytes)) + 1)
        sbuf = dev.alloc(sets * B * state_bytes)
        init = (rng.normal(0, 1, (B, vh, d, d)) * 0.1).astype(np.float32)
        for k in range(sets):
            call("pgd_device_memcpy", dev.handle, C.c_void_p(sbuf + k * B * state_bytes), init.ctypes.data_as(C.c_void_p),
                 C.c_size_t(init.nbytes), 0)
        ptrs = [dev.upload(np.array([sbuf + (k * B + i) * state_bytes for i in range(B)], np.uint64))
                for k in range(sets)]
        rs = dev.upload((np.arange(B) * toks).astype(np.int32))
        rc = dev.upload(np.full(B, toks, np.int32))
        o = dev.alloc(rows * vh * d * 4)

        def step(k):
            call("pgd_gdn_step_dev", dev.handle, kh, vh, *[C.c_void_p(p) for p in (conv, a, b, z, a_log, dtb, norm)],
                 C.c_void_p(ptrs[k]), C.c_void_p(rs), C.c_void_p(rc), B, C.c_void_p(o))

        for k in range(sets):
            step(k)
        L = max(32, 2 * sets)
        e0 = Event(dev).record()
        for i in range(L):
            step(i % sets)
        e1 = Event(dev).record()
        us = e0.elapsed_ms(e1) / L * 1e3
        algo = 2 * B * state_bytes + rows * (2 * kh * d + vh * d + 2 * vh + vh * d + vh * d) * 4
        gbs = algo / (us * 1e-6) / 1e9
        log(f"gdn B={B:2d} tokens={toks}: {us:8.2f} us {gbs:7.0f} GB/s {100 * gbs / HBM_PEAK_GBS:5.1f}%")
        out["gdn"].append({"B": B, "tokens": toks, "us": round(us, 3), "algo_bytes": algo, "gbs": round(gbs, 1),
                           "frac": round(gbs / HBM_PEAK_GBS, 4)})
        for p in [conv, a, b, z, a_log, dtb, norm, sbuf, rs, rc, o] + ptrs:
            dev.free(p)
    dev.close()
    return out


A8_SHAPES = [("gdn_in", 12352, 5120, 0), ("gdn_out", 5120, 4096, 1), ("attn_qkv", 14336, 5120, 0),
             ("attn_o", 5120, 6144, 1), ("down", 5120, 17408, 1), ("gateup", 17408, 5120, 2),
             ("lm_head", 151936, 5120, 0)]


def a8_sweep(rows_list, only=None):
    """Every config-4 A8 GEMV shape (epilogue as in the decode step: store,
    residual or fused SwiGLU) at the given row counts, prepared activations,
    HIP-event timed over launches cycling through weight copies that exceed
    the last-level cache (so every launch streams from HBM)."""
    from pagoda_amd import Device, Event, Matrix
    from pagoda_amd.matrix import act_bytes, act_prep_dev

    dev = Device(os.environ.get("PAGODA_DEVICE", "hip"))
    rng = np.random.default_rng(1)
    out = []
    for name, N, K, epi in A8_SHAPES:
        if only and name not in only:
            continue
        per = N * K * 8.5 / 8 * (2 if epi == 2 else 1)
        ncopy = max(2, int(1.6e9 // per) + 1)
        ms = [Matrix.synth(dev, 0, N, K, 7 + i, i * 16 + 1) for i in range(ncopy)]
        us = [Matrix.synth(dev, 0, N, K, 7 + i, i * 16 + 2) for i in range(ncopy)] if epi == 2 else None
        for rows in rows_list:
            x = dev.upload(rng.normal(0, 1, (rows, K)).astype(np.float32))
            act = dev.alloc(act_bytes(rows, K))
            y = dev.alloc(rows * N * 4)
            res = dev.alloc(rows * N * 4)
            act_prep_dev(dev, x, K, rows, K, act)

            def run(i):
                if epi == 2:
                    Matrix.gemv_swiglu_act_dev(ms[i], us[i], act, rows, y, N)
                elif epi == 1:
                    ms[i].gemv_act_dev(act, rows, y, N, res, N)
                else:
                    ms[i].gemv_act_dev(act, rows, y, N)

            for i in range(ncopy):
                run(i)
            L = max(24, 2 * ncopy)
            e0 = Event(dev).record()
            for i in range(L):
                run(i % ncopy)
            e1 = Event(dev).record()
            t_us = e0.elapsed_ms(e1) / L * 1e3
            algo = per + rows * K * 4 + rows * N * 4
            gbs = algo / (t_us * 1e-6) / 1e9
            flops = 2.0 * rows * N * K * (2 if epi == 2 else 1)
            tfs = flops / (t_us * 1e-6) / 1e12
            log(f"{name:9s} N={N:6d} K={K:5d} rows={rows:2d}: {t_us:8.1f} us {gbs:7.0f} GB/s {100 * gbs / HBM_PEAK_GBS:5.1f}%"
                f"  {tfs:6.1f} TFLOP/s useful")
            out.append({"matrix": name, "N": N, "K": K, "rows": rows, "us": round(t_us, 2), "algo_bytes": algo,
                        "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "useful_tflops": round(tfs, 1)})
            for p in (x, act, y, res):
                dev.free(p)
        for m in ms + (us or []):
            m.free()
    dev.close()
    return out


def config5_only():
    from pagoda_amd import Device
    from pagoda_amd.engine import QWEN35_27B, Model

    dev = Device(os.environ.get("PAGODA_DEVICE", "hip"))
    cfg = replace(QWEN35_27B, max_pos=C5_TRUNK + C5_SUFFIX + C5_GEN + 64, kv_blocks=C5_PAGES + 16)
    model = Model.synth(dev, cfg, seed=2026)
    out = config5(model, cfg)
    model.free()
    return out


def attn_scan():
    """Paged GQA decode attention alone (config-4 heads: 24 q / 4 kv, head_dim
    256), 1 and 32 rows, contexts of 40..4096 positions, 5 calls each through
    pgd_attn_decode_dev; every row reads its own pages."""
    import ctypes as C

    from pagoda_amd import Device
    from pagoda_amd._lib import call

    dev = Device(os.environ.get("PAGODA_DEVICE", "hip"))
    heads, kvh, hd, block = 24, 4, 256, 16
    rng = np.random.default_rng(0)
    for rows in (1, 32):
        for L in (40, 256, 1024, 4096):
            nb = (L + block - 1) // block
            pages = rows * nb + 1
            bufs = [dev.upload(rng.normal(0, 1, (rows, heads, hd)).astype(np.float32)),
                    dev.upload(rng.normal(0, 1, (rows, heads, hd)).astype(np.float32)),
                    dev.upload(rng.normal(0, 1, (pages, kvh, block, hd)).astype(np.float32)),
                    dev.upload(rng.normal(0, 1, (pages, kvh, block, hd)).astype(np.float32)),
                    dev.upload(np.arange(rows, dtype=np.int32)),
                    dev.upload(np.full(rows, L - 1, np.int32)),
                    dev.upload(np.arange(rows * nb, dtype=np.int32).reshape(rows, nb))]
            out = dev.alloc(rows * heads * hd * 4)
            for _ in range(5):
                call("pgd_attn_decode_dev", dev.handle, heads, kvh, hd, block, *[C.c_void_p(p) for p in bufs], nb,
                     rows, C.c_void_p(out))
            log(f"attn scan: rows={rows} positions={L}")
            for p in bufs + [out]:
                dev.free(p)


def copy_calib():
    """A plain device-to-device copy kernel of known size (256 MiB read +
    256 MiB written per launch) for scaling FETCH_SIZE / WRITE_SIZE."""
    import torch

    n = 256 << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(20):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": 20}), flush=True)


def cpu_baseline(args):
    """The oracle (C, OpenMP) on one full-width 3:1 layer group with a
    reduced vocab, per decode token, extrapolated by weight bytes to the
    64-layer model + full lm_head."""
    from oracle import pyoracle as ora

    cores = ora.lib().ora_num_threads()
    cpu_model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    c = ora.Qwen35Config(n_layers=4, vocab=4096)
    t0 = time.time()
    m = ora.Qwen35(c, 2026)
    log(f"cpu oracle: 4-layer group built in {time.time() - t0:.1f}s on {cores} threads")
    cache = m.new_cache()
    rng = np.random.default_rng(0)
    m.forward(rng.integers(0, c.vocab, 4), cache)
    n = 0
    t0 = time.perf_counter()
    tok = 1
    while n < 3 or (time.perf_counter() - t0 < 12.0 and n < 200):
        logits = m.forward([tok], cache)
        tok = int(np.argmax(logits))
        n += 1
    per_tok4 = (time.perf_counter() - t0) / n
    H, I, V = 5120, 17408, 151936
    lin = H * (8192 + 4096 + 64) + 4096 * H
    full = H * (12288 + 2048) + 6144 * H
    mlp = 3 * H * I
    group = (3 * lin + full + 4 * mlp) * 8.5 / 8
    small = group + 4096 * H * 8.5 / 8
    rate = small / per_tok4  # algorithmic weight bytes per second
    model_bytes = 16 * group + V * H * 8.5 / 8
    tok_s = rate / model_bytes
    return {"value": tok_s, "unit": "tok/s", "cores": cores, "kind": "port", "cpu_model": cpu_model,
            "host_cpus": os.cpu_count(),
            "sample": f"oracle.c decode, batch 1, one full-width 4-layer group (3 GDN + 1 attention, vocab 4096), "
                      f"{n} tokens in {per_tok4 * n:.1f}s; weight-bytes rate {rate / 1e9:.2f} GB/s extrapolated "
                      f"to 64 layers + 151936-row lm_head"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graphs", action="store_true", help="skip the graph-replayed passes (for kernel traces)")
    ap.add_argument("--roofline-only", action="store_true")
    ap.add_argument("--copy-calib", action="store_true")
    ap.add_argument("--no-config5", action="store_true")
    ap.add_argument("--config5-only", action="store_true",
                    help="run only the config-5 passes (for kernel traces of that workload)")
    ap.add_argument("--config1-only", action="store_true",
                    help="run only the config-1 passes (for kernel traces of that workload)")
    ap.add_argument("--attn-scan", action="store_true",
                    help="time the paged attention alone over context lengths (for kernel traces)")
    ap.add_argument("--a8-sweep", default=None, metavar="ROWS",
                    help="time every config-4 A8 GEMV shape at these row counts (e.g. 1,16,32,64)")
    ap.add_argument("--a8-only", default=None, metavar="NAMES", help="restrict --a8-sweep to these matrices")
    ap.add_argument("--kernel-sweeps", action="store_true",
                    help="config 2 (Q4_K/Q6_K GEMV sweep) and config 3 (GDN step) kernel timings")
    args = ap.parse_args()
    global USE_GRAPHS
    USE_GRAPHS = not args.no_graphs
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    if args.copy_calib:
        copy_calib()
        return
    if args.config5_only:
        print(json.dumps({"config5": config5_only()}), flush=True)
        return
    if args.config1_only:
        from pagoda_amd import Device

        dev = Device(os.environ.get("PAGODA_DEVICE", "hip"))
        print(json.dumps({"config1": config1(dev)}), flush=True)
        dev.close()
        return
    if args.attn_scan:
        attn_scan()
        return
    if args.a8_sweep:
        rows = [int(r) for r in args.a8_sweep.split(",")]
        only = args.a8_only.split(",") if args.a8_only else None
        print(json.dumps({"a8_sweep": a8_sweep(rows, only)}), flush=True)
        return
    if args.kernel_sweeps:
        print(json.dumps(kernel_sweeps()), flush=True)
        return
    if args.roofline_only:
        from pagoda_amd import Device
        from pagoda_amd.engine import QWEN35_27B

        print(json.dumps(roofline(Device(os.environ.get("PAGODA_DEVICE", "hip")), QWEN35_27B, args.batch)), flush=True)
        return
    g = gpu_bench(args)
    cpu = None if args.no_cpu else cpu_baseline(args)
    out = {
        "metric": "decode tok/s at batch 1 & 32; quant-GEMV HBM GB/s as % of MI355X peak",
        "value": round(g["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "dtype_note": ("fp32 accumulation and fp32 state/KV; A8 weight codes and activations enter the matrix "
                       "cores as f16 (activations as an f16 hi + lo pair, ~22 bits of the f32 value)"),
        "data": "synthetic (seeded random-init weights, random 19-token prompts)",
        "config": {"workload": "config4: 27B-class hybrid (64 layers, 3:1 GDN:attention), MLX affine-8, "
                               "greedy decode", "batch": args.batch, "prompt_len": 19,
                   "weight_gb": round(g["weight_gb"], 3), "algo_weight_gb_per_step": round(g["algo_gb_per_step"], 3)},
        "batch1_tok_s": round(g["batch1_tok_s"], 2),
        "graphs": None if g["tok_s_graph"] is None else {
                   "value": round(g["tok_s_graph"], 2), "batch1_tok_s": round(g["batch1_tok_s_graph"], 2),
                   "note": "the same decode steps replayed from HIP graphs (pgd_model_set_graphs), one per "
                           "launch signature; results bitwise equal to eager launches"},
        "step_ms_percentiles": g["step_ms_pct"],
        "config5": g["config5"],
        "config1": g["config1"],
        "roofline": g["roofline"],
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
