#!/usr/bin/env python3
"""bench.py — greedy decode throughput of the MI355X path on the reference's
headline workload (benchmark configuration C3): a Llama-3-8B-shape decoder (32 layers,
d 4096, 32 query / 8 kv heads of 128, SwiGLU FFN 14336, vocab 128256, RoPE
θ 500000) with seeded random-init Q4_K weights and a Q6_K output head, fp16
paged K/V prefilled to 2048 positions from random tokens, then greedy decode
at batch 1.

One "step" is one greedy token of the graph-captured decode step. W untimed
warmup steps run first, then exactly K timed steps bracketed by device
synchronisation; the model's weights, K/V and token history are resident in
HBM throughout (the decode loop hands nothing to the host inside the timed
region).

Beside the line's value it reports
  roofline      the dominant kernel (the fused gate|up Q4_K GEMV) timed with
                HIP events over back-to-back launches on the engine's
                stream, rotating over the 32 layers' weights (2.1 GB, past
                the 256 MB last-level cache): algorithmic bytes per launch ÷
                mean launch time, against 8 TB/s; `traffic` is the measured
                HBM bytes per launch from the committed rocprofv3 counter
                summary; `in_step_eager` the same launch timed inside whole
                eagerly enqueued decode steps (an event before and after each
                layer's launch: the kernel as the step runs it, plus its
                eager dispatch — an upper bound on its share of the graph-
                replayed step);
  copy          a plain 1 GiB device copy kernel (cj_buf_copy) timed the same
                way: the practical streaming ceiling of the part, and the
                known-size kernel the counter summaries are calibrated with;
  step_roofline the whole step: algorithmic bytes per token (weights at their
                GGUF size + K/V read + activation vectors) ÷ ms per step;
  cpu_baseline  the C restatement of the reference CPU backend (oracle/),
                OpenMP over the host cores, on a bounded sample of the same
                model's decode.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import re
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "decode tok/s, Llama-3-8B-shape Q4_K bs=1; achieved HBM GB/s as % of 8 TB/s"
PEAK_HBM_GBS = 8000.0
WORKLOAD = ("C3: Llama-3-8B shape (32 layers, d 4096, 32/8 heads of 128, FFN 14336, vocab 128256), "
            "Q4_K weights + Q6_K head, fp16 paged K/V, greedy, batch 1")
TRAFFIC_FILE = os.path.join(HERE, "profiles", "traffic_gemv_q4k_gate_up_c3.txt")
K_GATE_UP = 4
KIND_NAMES = {0: "embed", 1: "qkv", 2: "attention", 3: "o", 4: "gate_up", 5: "down", 6: "router", 7: "route",
              8: "expert_gate_up", 9: "expert_down", 10: "combine", 11: "head", 12: "norm", 13: "attn_merge"}
COPY_BYTES = 1 << 30          # the streaming-copy reference: 1 GiB read + 1 GiB written


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed counter
    summary (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", f.read(), re.M)
        return int(m.group(1)) if m else None
    except OSError:
        return None


def copy_reference(native, reps=20):
    """Mean time of a plain 1 GiB device-to-device copy (cj_buf_copy)."""
    lib = native.lib()
    src, dst = native.Buffer(COPY_BYTES), native.Buffer(COPY_BYTES)
    try:
        src.zero()
        native.check(lib.cj_buf_copy(dst.h, src.h, COPY_BYTES), "copy")
        native.sync()
        t0 = time.perf_counter()
        for _ in range(reps):
            native.check(lib.cj_buf_copy(dst.h, src.h, COPY_BYTES), "copy")
        native.sync()
        us = (time.perf_counter() - t0) * 1e6 / reps
    finally:
        src.free()
        dst.free()
    moved = 2 * COPY_BYTES
    return {"kernel": "cj_copy", "avg_us": round(us, 2), "bytes": moved, "GB/s": round(moved / (us * 1e-6) / 1e9, 1)}


def token_macs(cfg, count):
    """Multiply-adds of one decode token of a model (GGUF-derived config) at
    `count` attended positions: (weights, attention)."""
    L, h, nh, nkv, hd = cfg["n_layers"], cfg["hidden"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"]
    proj = h * (nh * hd + 2 * nkv * hd) + nh * hd * h
    if cfg["n_experts"]:
        ffn = cfg["n_experts"] * h + cfg["n_used"] * 3 * h * cfg["expert_ffn"]
    else:
        ffn = 3 * h * cfg["ffn"]
    weights = L * (proj + ffn) + cfg["vocab"] * h
    attn = 0
    for layer in range(L):
        w = cfg["swa_window"] if cfg["swa_window"] and (layer + 1) % max(1, cfg["swa_pattern"]) else 0
        attn += 2 * nh * hd * (min(w, count) if w else count)
    return weights, attn


def cpu_baseline(pkg, image_name, vocab, budget_s, seed, context, kv_f32=False):
    """Time the oracle's decode of the same model on the host cores: tokens
    at positions 1, 2, ... until `budget_s` of work is done (at least 2).
    The benchmarked context adds its attention's multiply-adds to the
    weights'; the rate there is estimated in proportion
    (`at_context_estimate`)."""
    from oracle import oracle as O
    from oracle.gguf_reader import GgufReader, oracle_model, model_config
    img = pkg.image_bytes(image_name)
    reader = GgufReader(img)
    om, _ = oracle_model(reader, ctx=64, kv_f32=kv_f32)
    try:
        rng = np.random.default_rng(seed + 1)
        toks = rng.integers(0, vocab, 64).tolist()
        om.step(toks[0], 0)                           # first touch of the weights, untimed
        n, t0 = 0, time.perf_counter()
        while n < 2 or (time.perf_counter() - t0 < budget_s and n < 62):
            om.step(toks[n + 1], n + 1)
            n += 1
        dt = time.perf_counter() - t0
    finally:
        om.close()
    cores = int(O.lib().or_model_threads())
    nproc, physical = host_cores()
    cfg = model_config(reader)
    w_short, a_short = token_macs(cfg, n // 2 + 1)
    w_ctx, a_ctx = token_macs(cfg, context)
    est = n / dt * (w_short + a_short) / (w_ctx + a_ctx)
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "nproc": nproc, "physical_cores": physical,
            "at_context_estimate": round(est, 3),
            "context": "sampled at positions 1..%d; at %d positions a token is %.3g G multiply-adds of weights and "
                       "%.3g G of attention (%.1f%%), so the rate there is estimated at %.3g tok/s"
                       % (n, context, w_ctx / 1e9, a_ctx / 1e9, 100.0 * a_ctx / (w_ctx + a_ctx), est),
            "sample": "%d greedy decode steps of the same C3 model at positions 1..%d (C restatement of the "
                      "reference CPU backend, oracle/oracle.c, OpenMP %d threads), %.1f s" % (n, n, cores, dt)}


def host_cores():
    """(logical CPUs this process may run on, physical cores of the host)."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        nproc = os.cpu_count() or 0
    cores, phys, core = set(), None, None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k == "physical id":
                    phys = v.strip()
                elif k == "core id":
                    core = v.strip()
                elif not k:
                    if core is not None:
                        cores.add((phys, core))
                    phys, core = None, None
        if core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    return nproc, len(cores) or None


C4_METRIC = "batched decode tok/s, Llama-3-8B-shape Q8_0, 32 seqs x 4096 ctx (prefill tok/s beside it)"
C4_WORKLOAD = ("C4: Llama-3-8B shape (32 layers, d 4096, 32/8 heads of 128, FFN 14336, vocab 128256), Q8_0 weights "
               "and head, fp16 paged K/V; batched greedy decode over 32 sequences at 4096 positions each; prefill "
               "of a 512-token chunk from position 0")


def run_c4(args, pkg, native):
    """Benchmark configuration C4: 32 sequences prefilled to `ctx` positions (prefill
    chunks of 512), then batched greedy decode of all 32 at once; and the
    prefill rate of one 512-token chunk from position 0."""
    nseq, ctx = args.seqs, args.ctx
    t = time.perf_counter()
    pkg.synth_gguf("c4", "mem:bench_c4", args.seed)
    log("synthesised C4 (seed %d) in %.1f s" % (args.seed, time.perf_counter() - t))
    opts = pkg.EngineOptions("mem:bench_c4")
    opts.ctx = ctx + args.warmup + args.steps + 1
    opts.maxSeqs = nseq
    opts.graphs = not args.eager
    t = time.perf_counter()
    eng = pkg.LlmEngine.load(opts)
    cfg = eng.config
    vocab = cfg["vocabSize"]
    log("loaded in %.1f s: %s" % (time.perf_counter() - t, cfg))
    rng = np.random.default_rng(args.seed)

    # prefill: one 512-token chunk from position 0, best of a few
    chunk = rng.integers(0, vocab, 512).tolist()
    pf = []
    for _ in range(args.prefill_reps):
        eng.reset(0)
        native.sync()
        t0 = time.perf_counter()
        eng.prefill(chunk, seq=0)
        native.sync()
        pf.append(time.perf_counter() - t0)
    log("prefill 512 rows: %s ms" % ", ".join("%.2f" % (x * 1e3) for x in pf))

    t = time.perf_counter()
    for s in range(nseq):
        eng.reset(s)
        eng.prefill(rng.integers(0, vocab, ctx).tolist(), seq=s)
    log("prefilled %d sequences x %d positions in %.1f s" % (nseq, ctx, time.perf_counter() - t))
    slots = list(range(nseq))
    eng.decodeBatch(slots, args.warmup)
    log("warmup %d batched steps: %.1f us/step" % (args.warmup, eng.lastStepMicros()))
    native.sync()
    t0 = time.perf_counter()
    out = eng.decodeBatch(slots, args.steps)
    native.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1000.0 / args.steps
    dev_us = eng.lastStepMicros()
    log("timed %d batched steps: %.3f ms/step wall, %.1f us/step device; %d distinct tokens"
        % (args.steps, ms_per_step, dev_us, len(set(out.ravel().tolist()))))

    # whole-step algorithmic bytes: the weights once, every sequence's K/V
    first = ctx + args.warmup
    kv_pos = cfg["numLayers"] * 2 * cfg["numKvHeads"] * cfg["headDim"] * 2
    one = np.mean([eng.stepBytes(int(c)) for c in range(first + 1, first + args.steps + 1)])
    step_bytes = float(one + (nseq - 1) * kv_pos * (first + 1 + args.steps / 2.0))
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        t = time.perf_counter()
        cpu = cpu_baseline(pkg, "bench_c4", vocab, args.cpu_seconds, args.seed, ctx + args.warmup + args.steps // 2)
        cpu["sample"] = cpu["sample"].replace("C3", "C4")
        log("cpu baseline: %s (%.1f s)" % (cpu, time.perf_counter() - t))
    eng.close()
    pkg.image_free("bench_c4")
    best = min(pf)
    line = {
        "metric": C4_METRIC,
        "value": round(nseq * args.steps / wall, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: seeded random-init GGUF (N(0,0.02) weights), uniform random prompt ids",
        "config": {"workload": C4_WORKLOAD, "batch": nseq, "prefill_positions": ctx,
                   "step": "eager launches" if args.eager else "hipGraph replay", "seed": args.seed},
        "prefill": {"value": round(512 / best, 1), "unit": "tok/s", "chunk": 512, "ms": round(best * 1e3, 3),
                    "reps_ms": [round(x * 1e3, 3) for x in pf]},
        "step_roofline": {"bytes_per_step": int(step_bytes), "achieved": round(step_gbs, 1), "peak": PEAK_HBM_GBS,
                          "unit": "GB/s", "frac": round(step_gbs / PEAK_HBM_GBS, 4),
                          "device_us_per_step": round(dev_us, 2)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


C2_METRIC = "quantised GEMV / mat-mat HBM GB/s (C2 microbench, cold weights)"
C2_FORMATS = (("q8_0", 8, 32, 34), ("q4_0", 2, 32, 18), ("q4_k", 12, 256, 144), ("q6_k", 14, 256, 210))
C2_SHAPES = ((4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096))
C2_BATCHES = (1, 4, 8, 16)
C2_POOL = 512 << 20


def c2_blocks(ty, nblocks, rng):
    """Random blocks of a format with sane scales (the f16 scale fields set,
    the rest random bytes), the shape of seeded N(0, 0.02) weights."""
    bb = {8: 34, 2: 18, 12: 144, 14: 210}[ty]
    raw = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)

    def f16(lo, hi):
        return rng.uniform(lo, hi, nblocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if ty in (8, 2):
        raw[:, 0:2] = f16(0.0005, 0.002)
    elif ty == 12:
        raw[:, 0:2] = f16(0.0001, 0.0005)
        raw[:, 2:4] = f16(0.0001, 0.0005)
    else:
        raw[:, 208:210] = f16(0.0001, 0.0003)
    return raw.reshape(-1)


def c2_cpu_baseline(seed, budget_s):
    """The oracle's Q4_K 14336x4096 mat-vec (C2's value row) timed on the host
    cores: repeated until `budget_s` of work is done (at least 3), rotating
    over 16 copies of the matrix (528 MB, past any host cache, as the GPU's
    pool is), weight GB/s."""
    from oracle import oracle as O
    rng = np.random.default_rng(seed + 2)
    rows, cols, copies = 14336, 4096, 16
    one = c2_blocks(12, rows * cols // 256, rng)
    pool = np.tile(one, copies).reshape(copies, -1)
    x = rng.standard_normal(cols).astype(np.float32)
    for c in range(copies):
        O.matvec(12, pool[c], rows, cols, x)          # first touch, untimed
    n, t0 = 0, time.perf_counter()
    while n < 3 or time.perf_counter() - t0 < budget_s:
        O.matvec(12, pool[n % copies], rows, cols, x)
        n += 1
    dt = time.perf_counter() - t0
    cores = int(O.lib().or_model_threads())
    nproc, physical = host_cores()
    return {"value": round(rows * cols // 256 * 144 * n / dt / 1e9, 3), "unit": "GB/s", "cores": cores,
            "kind": "port", "nproc": nproc, "physical_cores": physical,
            "sample": "%d mat-vecs of a Q4_K 14336x4096 matrix at batch 1 over 16 copies (pack + block dots, C "
                      "restatement of the reference CPU backend, oracle/oracle.c, OpenMP %d threads), %.1f s"
                      % (n, cores, dt)}


def run_c2(args, native):
    """Benchmark configuration C2: each format × shape × batch, weights rotated over a
    pool of >= 512 MB of distinct prepared copies so the 256 MB last-level
    cache cannot serve them; one captured graph of launches, timed whole.
    Batch 1 is the decode GEMV; batch > 1 the int8 matrix-core product where
    the format has one (Q8_0, Q4_K; Q6_K above 8 columns), else the
    many-column GEMV (Q6_K over packs, Q4_0 over the f32 columns)."""
    lib = native.lib()
    rng = np.random.default_rng(args.seed)
    table = []
    for fname, ty, be, bb in C2_FORMATS:
        for rows, cols in C2_SHAPES:
            wbytes = rows * cols // be * bb
            ncopy = max(2, -(-C2_POOL // wbytes))
            prb = lib.cj_prepared_row_bytes(ty, cols)
            raw = native.Buffer.of(c2_blocks(ty, rows * cols // be, rng))
            pool = native.Buffer(ncopy * rows * prb)
            for i in range(ncopy):
                native.check(lib.cj_prepare_weight(pool.h + i * rows * prb, raw.h, ty, rows, cols), "prepare")
            raw.free()
            bmax = max(C2_BATCHES)
            npad = (cols + 255) // 256 * 256
            xs = npad // 256 * 320
            x = rng.standard_normal((bmax, cols)).astype(np.float32)
            xb = native.Buffer.of(x)
            xp = native.Buffer(bmax * xs)
            native.check(lib.cj_q8k_pack(xp.h, xb.h, bmax, cols, npad, int(ty == 8)), "pack")
            y = native.Buffer(bmax * rows * 4)
            f32act = ty == 2
            for B in C2_BATCHES:
                reps = max(ncopy, 32)
                native.check(lib.cj_graph_begin(), "graph")
                for r in range(reps):
                    w = pool.h + (r % ncopy) * rows * prb
                    if B == 1:
                        act = xb.h if f32act else xp.h
                        native.check(lib.cj_matvec(ty, y.h, w, act, rows, cols, 0, 0), "matvec")
                    elif f32act:
                        native.check(lib.cj_matmul(ty, y.h, w, xb.h, rows, cols, B, cols * 4, rows, 0, 0), "matmul")
                    else:
                        native.check(lib.cj_matmul(ty, y.h, w, xp.h, rows, cols, B, xs, rows, 0, 0), "matmul")
                g = native.handle(lib.cj_graph_end(), "graph")
                native.check(lib.cj_graph_launch(g), "graph launch")
                native.sync()
                t0 = time.perf_counter()
                native.check(lib.cj_graph_launch(g), "graph launch")
                native.sync()
                us = (time.perf_counter() - t0) * 1e6 / reps
                lib.cj_graph_free(g)
                nbytes = wbytes + B * cols * 4 + B * rows * 4
                gbs = nbytes / (us * 1e-6) / 1e9
                table.append({"format": fname, "rows": rows, "cols": cols, "batch": B, "us": round(us, 2),
                              "bytes": nbytes, "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4),
                              "kernel": "gemv" if B == 1 else ("many-column gemv" if ty == 2 or (ty == 14 and B <= 8) else "int8 mfma"),
                              "pool_copies": ncopy})
                log("  %-5s %6d x %5d B %2d: %9.2f us  %7.1f GB/s  (%s, %d copies)" % (
                    fname, rows, cols, B, us, gbs, table[-1]["kernel"], ncopy))
            for b in (pool, xb, xp, y):
                b.free()
    head = next(t for t in table if t["format"] == "q4_k" and t["rows"] == 14336 and t["batch"] == 1)
    line = {
        "metric": C2_METRIC,
        "value": head["GB/s"],
        "unit": "GB/s",
        "n_gpus": 1, "steps": None, "warmup": 1, "ms_per_step": None, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: seeded random blocks (sane f16 scales), activations N(0, 1)",
        "config": {"workload": "C2: quantised GEMV microbench; value = Q4_K 14336x4096 at batch 1",
                   "formats": [f[0] for f in C2_FORMATS], "shapes": C2_SHAPES, "batches": C2_BATCHES,
                   "cold_pool_bytes": C2_POOL},
        "roofline": {"bound": "hbm", "achieved": head["GB/s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": head["frac"], "traffic": None},
        "table": table,
        "cpu_baseline": None if args.no_cpu else c2_cpu_baseline(args.seed, args.cpu_seconds),
    }
    print(json.dumps(line), flush=True)


SINGLE = {
    # workload: (synth spec, prompt positions, timed steps, metric, workload text)
    "c1": ("c1", 16, 64, "decode us/token, tiny Llama Q8_0 (C1), batch 1",
           "C1: 4 layers, d 512, 8/2 heads of 64, FFN 1408, vocab 32000, Q8_0 weights, f32 embeddings; "
           "16-token prompt, 64 greedy tokens"),
    "c5": ("c5", 4096, 64, "decode tok/s, gpt-oss-20b-shape MXFP4 MoE, batch 1, 4096 context",
           "C5: 24 layers, d 2880, 64/8 heads of 64, 32 MXFP4 experts top-4 of FFN 2880, alternating "
           "128-window attention, vocab 201088; fp16 paged K/V prefilled to 4096 positions, greedy"),
}


def run_single(args, pkg, native, which):
    """C1 and C5: one sequence, prompt then greedy decode through the graph-
    replayed step, as the headline does for C3."""
    spec, ctx, steps, metric, workload = SINGLE[which]
    ctx = args.ctx or ctx
    steps = steps if args.steps == 256 else args.steps
    name = "bench_" + which
    t = time.perf_counter()
    pkg.synth_gguf(spec, "mem:" + name, args.seed)
    log("synthesised %s (seed %d) in %.1f s" % (which.upper(), args.seed, time.perf_counter() - t))
    opts = pkg.EngineOptions("mem:" + name)
    opts.ctx = ctx + args.warmup + steps + 1
    opts.maxSeqs = 1
    opts.graphs = not args.eager
    opts.cpuThreads = args.cpu_threads
    opts.kvF32 = args.kv == "f32"
    eng = pkg.LlmEngine.load(opts)
    vocab = eng.config["vocabSize"]
    rng = np.random.default_rng(args.seed)
    t = time.perf_counter()
    eng.reset()
    eng.prefill(rng.integers(0, vocab, ctx).tolist())
    log("prefilled %d positions in %.1f s" % (ctx, time.perf_counter() - t))
    eng.decode(args.warmup)
    native.sync()
    t0 = time.perf_counter()
    toks = eng.decode(steps)
    native.sync()
    wall = time.perf_counter() - t0
    us_tok = wall * 1e6 / steps
    log("timed %d steps: %.1f us/token wall, %.1f us/step device; %d distinct tokens"
        % (steps, us_tok, eng.lastStepMicros(), len(set(int(x) for x in toks))))
    first = ctx + args.warmup
    step_bytes = float(np.mean([eng.stepBytes(int(c)) for c in range(first + 1, first + steps + 1)]))
    step_gbs = step_bytes / (us_tok * 1e-6) / 1e9
    kernels = {}
    for kind, kname in sorted(KIND_NAMES.items()):
        try:
            us, nbytes, kn = eng.timeKernel(kind, args.kernel_reps)
        except pkg.LlmException as e:
            if "launches nothing" not in str(e) and "not part of" not in str(e):
                raise
            continue
        kernels[kname] = {"kernel": kn, "avg_us": round(us, 3), "bytes": nbytes,
                          "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1)}
        log("  %-13s %-26s %9.2f us  %12d B  %7.1f GB/s" % (kname, kn, us, nbytes, nbytes / (us * 1e-6) / 1e9))
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(pkg, name, vocab, args.cpu_seconds, args.seed, ctx + args.warmup + steps // 2,
                           kv_f32=args.kv == "f32")
        cpu["sample"] = cpu["sample"].replace("C3", which.upper())
        log("cpu baseline: %s" % cpu)
    eng.close()
    pkg.image_free(name)
    c1 = which == "c1"
    line = {
        "metric": metric,
        "value": round(us_tok, 2) if c1 else round(steps / wall, 2),
        "unit": "us/token" if c1 else "tok/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "ms_per_step": round(us_tok / 1e3, 4),
        "higher_is_better": not c1, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: seeded random-init GGUF (N(0,0.02) weights), uniform random prompt ids",
        "config": {"workload": workload + ("; f32 K/V cache (PagedKvCache's mode, as the config states it)"
                                           if args.kv == "f32" else "; fp16 paged K/V"),
                   "batch": 1, "prefill_positions": ctx, "kv": args.kv,
                   "step": "eager launches" if args.eager else "hipGraph replay", "seed": args.seed},
        "step_roofline": {"bytes_per_token": int(step_bytes), "achieved": round(step_gbs, 1), "peak": PEAK_HBM_GBS,
                          "unit": "GB/s", "frac": round(step_gbs / PEAK_HBM_GBS, 4),
                          "wall_us_per_step": round(us_tok, 2)},
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


C5B_METRIC = "batched decode tok/s, gpt-oss-20b-shape MXFP4 MoE, 16 seqs x 4096 ctx"


def run_c5_batch(args, pkg, native):
    """Benchmark configuration C5 at batch > 1: `seqs` sequences prefilled to `ctx`
    positions (prefill chunks of decode-attention rows), then batched greedy
    decode of all of them through the captured batch step; beside it the
    same engine's batch-1 step on one of the sequences, for the per-token
    comparison with decoding the sequences one at a time."""
    nseq, ctx = args.seqs, args.ctx or 4096
    steps = 32 if args.steps == 256 else args.steps
    t = time.perf_counter()
    pkg.synth_gguf("c5", "mem:bench_c5b", args.seed)
    log("synthesised C5 (seed %d) in %.1f s" % (args.seed, time.perf_counter() - t))
    opts = pkg.EngineOptions("mem:bench_c5b")
    opts.ctx = ctx + 2 * (args.warmup + steps) + 1
    opts.maxSeqs = nseq
    opts.graphs = not args.eager
    eng = pkg.LlmEngine.load(opts)
    cfg = eng.config
    vocab = cfg["vocabSize"]
    log("loaded: %s" % cfg)
    rng = np.random.default_rng(args.seed)
    t = time.perf_counter()
    for s in range(nseq):
        eng.reset(s)
        eng.prefill(rng.integers(0, vocab, ctx).tolist(), seq=s)
    native.sync()
    pf_s = time.perf_counter() - t
    log("prefilled %d sequences x %d positions in %.1f s (%.0f tok/s)" % (nseq, ctx, pf_s, nseq * ctx / pf_s))
    slots = list(range(nseq))
    eng.decodeBatch(slots, args.warmup)
    native.sync()
    t0 = time.perf_counter()
    out = eng.decodeBatch(slots, steps)
    native.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1000.0 / steps
    dev_us = eng.lastStepMicros()
    log("timed %d batched steps of %d rows: %.3f ms/step wall, %.1f us/step device; %d distinct tokens"
        % (steps, nseq, ms_per_step, dev_us, len(set(out.ravel().tolist()))))
    # the batch-1 step of slot 0 (the same positions' cost, one sequence a step)
    eng.decode(args.warmup, seq=0)
    native.sync()
    t0 = time.perf_counter()
    eng.decode(steps, seq=0)
    native.sync()
    one_ms = (time.perf_counter() - t0) * 1000.0 / steps
    log("batch-1 step of the same model: %.3f ms/token; batched: %.3f ms/token (%.1fx)"
        % (one_ms, ms_per_step / nseq, one_ms / (ms_per_step / nseq)))
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(pkg, "bench_c5b", vocab, args.cpu_seconds, args.seed, ctx + args.warmup + steps // 2)
        cpu["sample"] = cpu["sample"].replace("C3", "C5")
        log("cpu baseline: %s" % cpu)
    eng.close()
    pkg.image_free("bench_c5b")
    line = {
        "metric": C5B_METRIC,
        "value": round(nseq * steps / wall, 2),
        "unit": "tok/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: seeded random-init GGUF (N(0,0.02) weights), uniform random prompt ids",
        "config": {"workload": "C5: gpt-oss-20b shape (24 layers, d 2880, 64/8 heads of 64, 32 MXFP4 experts "
                               "top-4 of FFN 2880, alternating 128-window attention, vocab 201088), batched "
                               "greedy decode", "batch": nseq, "prefill_positions": ctx,
                   "step": "eager launches" if args.eager else "hipGraph replay", "seed": args.seed},
        "batch1": {"ms_per_token": round(one_ms, 4), "speedup_per_token": round(one_ms / (ms_per_step / nseq), 2)},
        "prefill": {"value": round(nseq * ctx / pf_s, 1), "unit": "tok/s", "positions": nseq * ctx},
        "device_us_per_step": round(dev_us, 2),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def run_c5k(args, native):
    """The C5 kernels at their shapes through the launch seam (weights
    prepared once with cj_prepare_weight, seeded random blocks): the expert
    products, the router and the two-pass attention at 4096 positions. Host
    launches back to back, timed over the batch of calls."""
    lib = native.lib()
    rng = np.random.default_rng(args.seed)
    out = {}
    for name, ty, rows, cols, bb, be in (("mxfp4 experts down 4x2880x2880", 39, 11520, 2880, 17, 32),
                                         ("mxfp4 experts gate|up 4x5760x2880", 39, 23040, 2880, 17, 32),
                                         ("f32 router 32x2880", 0, 32, 2880, 4, 1)):
        raw = rng.integers(0, 256, rows * cols // be * bb, dtype=np.uint8)
        if ty == 0:
            raw = rng.standard_normal(rows * cols).astype(np.float32).view(np.uint8)
        else:
            r = raw.reshape(-1, bb)
            r[:, 0] = rng.integers(110, 130, r.shape[0])
        prb = lib.cj_prepared_row_bytes(ty, cols)
        src, w = native.Buffer.of(raw), native.Buffer(prb * rows)
        native.check(lib.cj_prepare_weight(w.h, src.h, ty, rows, cols), "prepare")
        x = native.Buffer.of(rng.standard_normal(cols).astype(np.float32))
        y = native.Buffer(rows * 4)
        for _ in range(5):
            native.check(lib.cj_matvec(ty, y.h, w.h, x.h, rows, cols, 0, 0), "matvec")
        native.sync()
        t = time.perf_counter()
        for _ in range(200):
            lib.cj_matvec(ty, y.h, w.h, x.h, rows, cols, 0, 0)
        native.sync()
        us = (time.perf_counter() - t) / 200 * 1e6
        out[name] = {"us": round(us, 2), "GB/s": round(prb * rows / (us * 1e-6) / 1e9, 1)}
        log("%-36s %8.2f us" % (name, us))
    n_q, n_kv, hd, count = 64, 8, 64, 4096
    pages = (count + 63) // 64
    kb = native.Buffer.of((rng.standard_normal(pages * n_kv * 64 * hd) * 0.5).astype(np.float16).view(np.uint16))
    vb = native.Buffer.of((rng.standard_normal(pages * n_kv * 64 * hd) * 0.5).astype(np.float16).view(np.uint16))
    tb = native.Buffer.of(np.arange(pages, dtype=np.int32))
    qb = native.Buffer.of(rng.standard_normal(n_q * hd).astype(np.float32))
    part = native.Buffer(n_q * max(64 * (hd + 2), count) * 4)
    ob, cnt = native.Buffer(n_q * hd * 4), native.Buffer(4 * n_kv)
    for _ in range(103):
        native.check(lib.cj_attend(part.h, ob.h, qb.h, kb.h, vb.h, tb.h, 0, cnt.h, n_q, n_kv, hd, count, 0, 512, 0.125),
                     "attend")
    native.sync()
    print(json.dumps({"metric": "C5 kernels at their shapes (launch seam; per-kernel durations from rocprofv3)",
                      "value": out["mxfp4 experts down 4x2880x2880"]["us"], "unit": "us", "n_gpus": 1,
                      "higher_is_better": False, "data": "synthetic: seeded random blocks",
                      "config": {"workload": "C5 kernel shapes"}, "kernels": out}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode steps (K)")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode steps before (W)")
    ap.add_argument("--workload", choices=("c3", "c4", "c2", "c1", "c5", "c5k"), default="c3",
                    help="c3: the headline batch-1 Q4_K decode; c4: batched Q8_0 decode + prefill; "
                         "c2: the quantised GEMV microbench; c1: tiny Q8_0 decode; c5: MoE decode; "
                         "c5k: the C5 kernels at their shapes through the launch seam")
    ap.add_argument("--ctx", type=int, default=None, help="positions prefilled before decoding (c3 2048, c4 4096)")
    ap.add_argument("--seqs", type=int, default=None,
                    help="sequences decoded together: c4 (default 32); c5 above 1 times the batched decode")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="the CPU worker count the attention split rule follows (0: the engine's 512)")
    ap.add_argument("--prefill-reps", type=int, default=3, help="c4: timed 512-row prefill chunks")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--kernel-reps", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--kv", choices=("f16", "f32"), default="f16",
                    help="c1: the K/V cache's element type (f32: BASELINE.json's C1 as stated)")
    ap.add_argument("--eager", action="store_true",
                    help="enqueue each step's launches instead of replaying the graph (for profilers)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one MI355X; --gpus %d (WORLD_SIZE %d) is not run. The decode step "
              "would shard by tensor parallelism across GPUs; nothing here uses a second GPU." % (args.gpus, world),
              file=sys.stderr)
        sys.exit(2)

    import __graft_entry__ as entry
    pkg = entry.load_package()
    from cajeta_llm_amd import native

    native.init()
    if args.workload == "c2":
        run_c2(args, native)
        return
    if args.workload == "c5k":
        run_c5k(args, native)
        return
    if args.workload == "c5" and (args.seqs or 1) > 1:
        run_c5_batch(args, pkg, native)
        return
    if args.workload in SINGLE:
        run_single(args, pkg, native, args.workload)
        return
    if args.workload == "c4":
        if args.ctx is None:
            args.ctx = 4096
        if args.steps == 256:
            args.steps = 32
        if args.seqs is None:
            args.seqs = 32
        run_c4(args, pkg, native)
        return
    if args.ctx is None:
        args.ctx = 2048
    t = time.perf_counter()
    pkg.synth_gguf("c3", "mem:bench_c3", args.seed)
    log("synthesised C3 (seed %d) in %.1f s" % (args.seed, time.perf_counter() - t))

    total = args.ctx + args.warmup + args.steps + 8    # room for the LlmEngine leg's request too
    opts = pkg.EngineOptions("mem:bench_c3")
    opts.ctx = total
    opts.maxSeqs = 1
    opts.graphs = not args.eager
    opts.cpuThreads = args.cpu_threads
    t = time.perf_counter()
    eng = pkg.LlmEngine.load(opts)
    cfg = eng.config
    vocab = cfg["vocabSize"]
    log("loaded in %.1f s: %s" % (time.perf_counter() - t, cfg))

    rng = np.random.default_rng(args.seed)
    prompt = rng.integers(0, vocab, args.ctx).tolist()
    t = time.perf_counter()
    eng.reset()
    eng.prefill(prompt)
    log("prefilled %d positions in %.1f s" % (args.ctx, time.perf_counter() - t))
    eng.decode(args.warmup)
    log("warmup %d steps: %.1f us/step" % (args.warmup, eng.lastStepMicros()))

    native.sync()
    t0 = time.perf_counter()
    toks = eng.decode(args.steps)
    native.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1000.0 / args.steps
    dev_us = eng.lastStepMicros()
    log("timed %d steps: %.3f ms/step wall, %.1f us/step device; %d distinct tokens"
        % (args.steps, ms_per_step, dev_us, len(set(int(x) for x in toks))))

    # whole-step algorithmic bytes over the timed positions
    first = args.ctx + args.warmup                     # position of the first timed step
    counts = np.arange(first + 1, first + args.steps + 1)
    step_bytes = float(np.mean([eng.stepBytes(int(c)) for c in counts]))
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9

    # per-kernel breakdown, the dominant one first
    kernels = {}
    for kind in (K_GATE_UP, 1, 2, 13, 3, 5, 12, 11, 0):
        try:
            us, nbytes, name = eng.timeKernel(kind, args.kernel_reps)
        except pkg.LlmException as e:
            if "launches nothing" not in str(e):
                raise
            continue
        kernels[KIND_NAMES[kind]] = {"kernel": name, "avg_us": round(us, 3), "bytes": nbytes,
                                     "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1)}
        log("  %-9s %-26s %9.2f us  %12d B  %7.1f GB/s" % (KIND_NAMES[kind], name, us, nbytes,
                                                           nbytes / (us * 1e-6) / 1e9))
    dom = kernels["gate_up"]
    achieved = dom["bytes"] / (dom["avg_us"] * 1e-6) / 1e9
    # the same kinds inside whole eager steps (every layer's launch between
    # two events; each interval holds the launch's share of the boundary)
    in_step = {}
    for kind in (K_GATE_UP, 1, 2, 3, 5):
        us = eng.timeKernelInStep(kind, 4)
        in_step[KIND_NAMES[kind]] = round(us, 3)
        log("  in step  %-9s %9.2f us" % (KIND_NAMES[kind], us))
    dom_in = in_step["gate_up"]
    copy = copy_reference(native)
    log("  copy      cj_copy                   %9.2f us  %12d B  %7.1f GB/s" % (copy["avg_us"], copy["bytes"],
                                                                              copy["GB/s"]))

    # the same decode through the LlmEngine surface: one greedy request,
    # stepOnce per token (the scheduler's pipelined step: the next token's
    # step is queued before the last one's token is read)
    api = None
    if not args.eager:
        rid = eng.submitTokens(prompt, maxNew=args.warmup + args.steps + 4, params=pkg.SampleParams(stopTokens=[]))
        for _ in range(2 + args.warmup):             # the prompt (its first token), the pipeline's seed, warmup
            eng.stepOnce()
        native.sync()
        n0 = len(eng.request(rid).tokens)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            eng.stepOnce()
        api_wall = time.perf_counter() - t0
        n1 = len(eng.request(rid).tokens)
        eng.cancel(rid)
        api = {"path": "LlmEngine.submitTokens + stepOnce (pipelined greedy step)", "tokens": n1 - n0,
               "ms_per_step": round(api_wall * 1000.0 / max(1, n1 - n0), 4),
               "tok/s": round((n1 - n0) / api_wall, 2), "vs_decode": round((n1 - n0) / api_wall / (args.steps / wall), 4)}
        log("api: %d tokens through stepOnce, %.3f ms/step (%.1f%% of the decode rate)"
            % (n1 - n0, api["ms_per_step"], 100 * api["vs_decode"]))

    cpu = None
    if not args.no_cpu:
        t = time.perf_counter()
        cpu = cpu_baseline(pkg, "bench_c3", vocab, args.cpu_seconds, args.seed, args.ctx + args.warmup + args.steps // 2)
        log("cpu baseline: %s (%.1f s)" % (cpu, time.perf_counter() - t))
    eng.close()
    pkg.image_free("bench_c3")

    line = {
        "metric": METRIC,
        "value": round(args.steps / wall, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: seeded random-init GGUF (N(0,0.02) weights), uniform random prompt ids",
        "config": {"workload": WORKLOAD, "batch": 1, "prefill_positions": args.ctx,
                   "step": "eager launches" if args.eager else "hipGraph replay",
                   "timed_positions": [first, first + args.steps - 1], "seed": args.seed},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": measured_traffic(),
                     "kernel": dom["kernel"], "bytes_per_launch": dom["bytes"], "avg_us": dom["avg_us"],
                     "in_step_eager": {"avg_us": dom_in, "achieved": round(dom["bytes"] / (dom_in * 1e-6) / 1e9, 1),
                                       "frac": round(dom["bytes"] / (dom_in * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                                       "note": "events around each layer's launch in eagerly enqueued steps: "
                                               "the kernel plus its eager dispatch (an upper bound on its "
                                               "share of the graph-replayed step)"}},
        "step_roofline": {"bytes_per_token": int(step_bytes), "achieved": round(step_gbs, 1),
                          "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(step_gbs / PEAK_HBM_GBS, 4),
                          "device_us_per_step": round(dev_us, 2)},
        "kernels": kernels,
        "kernels_in_step_eager_us": in_step,
        "copy": copy,
        "api": api,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
