#!/usr/bin/env python3
"""Q8 decode benchmark on one MI355X: Mistral-7B shape, batch 1.

Workload (the configuration the headline metric is quoted on): a
Mistral-7B-shape decoder (hidden 4096, 32 layers, 32 query / 8 KV heads,
SwiGLU 14336, vocab 32768, untied head) with seeded N(0, 0.02) weights
packed to Q8 on the device, a 128-token uniform-random prompt prefilled in
one chunk, then greedy decode (graph-replayed steps, device argmax) with
32-token KV pages.  One step = one decode token.  --warmup W steps run
untimed, then exactly --steps K steps are timed with HIP events on the
executor's stream (bracketed by stream synchronisation).

Reported:
  value          weight bytes streamed per decode token x tokens/s (GB/s)
  roofline       the decode step's dominant kernel, the Q8 dequant-GEMV over
                 the fused gate/up storage (28672 x 4096), batch 1:
                 back-to-back launches over the 32 layers' matrices (3.8 GB,
                 far beyond the 256 MB MALL) between one pair of HIP events
                 on the launch stream; gemv_14336x4096 gives the same for
                 the up projection alone
  cpu_baseline   the oracle (C restatement of the reference's Go CPU path)
                 decoding a few tokens of the same model on the host cores
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
PROMPT, TOKENS = 128, 256
# Reference receipt for the same workload: Mistral-7B Q8 decode, batch 1,
# Apple M4, GOMAXPROCS=4: 0.750 s/token = 1.33 tok/s = 10.1 GB/s of weights.
REF_GBS = 10.1


class HipEvents:
    """hipEventCreate/Record/ElapsedTime on an explicit stream."""

    def __init__(self):
        self.hip = C.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [C.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]

    def create(self):
        e = C.c_void_p()
        assert self.hip.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, ev, stream):
        assert self.hip.hipEventRecord(ev, stream) == 0

    def elapsed_ms(self, a, b):
        assert self.hip.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.hip.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return ms.value

    def destroy(self, ev):
        self.hip.hipEventDestroy(ev)


def gemv_roofline(srq, ex, weights, hip, launches, label):
    """Time the Q8 / Q4 GEMV (batch 1) over `weights`: `launches`
    back-to-back launches cycling over the distinct matrices (together far
    larger than the 256 MB MALL), one HIP event pair on the launch stream
    around all of them."""
    rows, cols, fmt = weights[0].rows, weights[0].cols, weights[0].fmt
    tag = {srq.Q8: "q8", srq.Q4: "q4"}[fmt]
    x = ex.empty(cols * 4)
    srq.fill_normal(ex, x, cols, 7, 1.0)
    y = ex.empty(rows * 4)
    stream = C.c_void_p(ex.stream)
    L = srq.lib()
    for w in weights[:4]:  # warm the code path
        srq.check(L.srq_linear_enqueue(ex.h, y.ptr, x.ptr, w.h, 1))
    ex.synchronize()
    a, b = hip.create(), hip.create()
    hip.record(a, stream)
    for i in range(launches):
        srq.check(L.srq_linear_enqueue(ex.h, y.ptr, x.ptr, weights[i % len(weights)].h, 1))
    hip.record(b, stream)
    ms = hip.elapsed_ms(a, b)
    ex.synchronize()
    hip.destroy(a)
    hip.destroy(b)
    vb, sb = srq.packed_bytes(fmt, rows, cols)
    algo = vb + sb + cols * 4 + rows * 4
    avg_s = ms / 1e3 / launches
    achieved = algo / avg_s / 1e9
    name = "gemv_%s_%dx%d" % (tag, rows, cols)
    prof_us = read_profile_avg_us(name + "_kernel_trace.txt",
                                  "void gemv_stream_kernel<%d, 1, 0, false, true," % fmt)
    return {
        "kernel": "gemv_stream_kernel<%s, n=1, plain> %dx%d (%s)" % (tag.upper(), rows, cols, label),
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": read_traffic(name + "_pmc.txt"),
        "algorithmic_bytes_per_launch": algo, "avg_launch_us": round(avg_s * 1e6, 3),
        "launches": launches,
        # the committed rocprofv3 summary of the standalone leg (its tracer
        # adds a little per dispatch): same bytes over its average duration
        "profile": None if prof_us is None else {
            "file": "profiles/%s_kernel_trace.txt" % name, "avg_kernel_us": prof_us,
            "frac": round(algo / (prof_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
    }


def gemv_only(srq, launches, seed, rows, fmt="q8"):
    """The roofline leg alone, for counter runs: standalone Q8 / Q4 weights
    rows x 4096 (about 2 GB of distinct packed matrices) packed on the
    device, `launches` GEMV launches, then one 256 MiB device-to-device copy
    whose known byte count calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    ex = srq.Executor(0)
    cols = 4096
    f = {"q8": srq.Q8, "q4": srq.Q4}[fmt]
    vb, sb = srq.packed_bytes(f, rows, cols)
    count = max(2, (2 << 30) // (vb + sb))
    src = ex.empty(rows * cols * 4)
    weights = []
    for i in range(count):
        srq.fill_normal(ex, src, rows * cols, seed * 7919 + i, 0.02)
        h = C.c_void_p()
        srq.check(srq.lib().srq_weight_create(ex.h, f, rows, cols, src.ptr, srq.SRC_F32, C.byref(h)))
        weights.append(srq.Weight(h))
    src.close()
    ex.synchronize()
    roof = gemv_roofline(srq, ex, weights, HipEvents(), launches, "standalone matrices")
    copy_bytes = 256 << 20
    a, b = ex.empty(copy_bytes), ex.empty(copy_bytes)
    srq.check(srq.lib().srq_copy_d2d(ex.h, b.ptr, a.ptr, copy_bytes))
    ex.synchronize()
    print(json.dumps({"roofline": roof, "calibration_copy_bytes": copy_bytes}), flush=True)
    return 0


def read_profile_avg_us(name, kernel_prefix):
    """Average duration (us) of the roofline kernel in a committed rocprofv3
    --kernel-trace --stats summary."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.strip().startswith(kernel_prefix):
                return float(line.split()[-3])
    except (OSError, ValueError, IndexError):
        pass
    return None


def read_traffic(name):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":")[1]))
    except OSError:
        pass
    return None


def cpu_baseline(srq, ex, model, cfg, cache, first, gpu_tokens, n_tokens):
    """Decode n_tokens of the same model with the oracle on the host."""
    import oracle
    t_setup = time.perf_counter()
    weights = {}

    def take(name, w):
        vals, scl = w.packed(ex)
        weights[name] = oracle.Weight(oracle.Q8, w.rows, w.cols, vals.view(np.int8).reshape(w.rows, w.cols),
                                      scl.reshape(w.rows, -1))

    take("embed_tokens", model.weight(srq.T_EMBED))
    take("lm_head", model.weight(srq.T_OUTPUT))
    names = {"q_proj": srq.T_Q, "k_proj": srq.T_K, "v_proj": srq.T_V, "o_proj": srq.T_O, "gate_proj": srq.T_GATE,
             "up_proj": srq.T_UP, "down_proj": srq.T_DOWN}
    ones = np.ones(cfg.dim, np.float32)
    for layer in range(cfg.layers):
        for nm, kind in names.items():
            take("layers.%d.%s" % (layer, nm), model.weight(kind, layer))
        for nm in ("input_layernorm", "post_attention_layernorm"):
            weights["layers.%d.%s" % (layer, nm)] = oracle.Weight(oracle.F32, 1, cfg.dim, ones)
    weights["norm"] = oracle.Weight(oracle.F32, 1, cfg.dim, ones)
    ocfg = oracle.make_config(cfg.vocab, cfg.dim, cfg.layers, cfg.heads, cfg.kv_heads, cfg.hidden, cfg.context,
                              cfg.rope_theta, cfg.norm_eps, False)
    om = oracle.Model(ocfg, weights)
    oc = om.new_cache()
    for layer in range(cfg.layers):
        k, v = cache.read(layer, 0, PROMPT)
        oc.set_rows(layer, 0, k, v)
    oc.set_pos(PROMPT)
    setup_s = time.perf_counter() - t_setup
    feed = [first] + gpu_tokens
    runs = []
    # All host cores (16 at most: the GPU box's CPU share), then 4 threads,
    # the GOMAXPROCS of the reference's published receipts.
    for workers, count in ((min(os.cpu_count() or 1, 16), n_tokens), (4, max(1, n_tokens // 4))):
        oc.set_pos(PROMPT)
        t0 = time.perf_counter()
        produced = []
        for i in range(count):
            logits = om.step([oc], [[feed[i]]], workers=workers)[0]
            produced.append(oracle.argmax(logits))
        runs.append((workers, count / (time.perf_counter() - t0), produced))
    om.close()
    return runs, setup_s


def host_facts():
    """nproc and CPU model of the host the CPU baseline runs on."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model or os.uname().machine}


def percentiles(us):
    a = np.sort(np.asarray(us, np.float64))
    return float(np.median(a)), float(a[int(0.1 * (len(a) - 1))]), float(a[int(0.9 * (len(a) - 1))])


def bench_smollm2(srq, args):
    """SmolLM2-135M architecture (576 / 30 layers / 9:3 heads / 1536 /
    49152 tied), Q8, seeded N(0, 0.02) weights: 32-token random prompt, then
    64 greedy tokens (graph-replayed decode).  Tokens/s over the 63 replayed
    decode steps of a second generation (the first warms the graph)."""
    from sr_go_tranformer_amd import synthetic
    ex = srq.Executor(0)
    cfg = synthetic.shape_config("smollm2-135m", 2048)
    model = synthetic.build(ex, cfg, "q8", args.seed)
    hip = HipEvents()
    stream = C.c_void_p(ex.stream)
    pool = model.pool(8)
    prompt = synthetic.random_prompt(32, cfg.vocab, args.seed)
    times, tokens = [], None
    for rep in range(3):
        cache = pool.cache(4)
        model.step([cache], [prompt])
        first = int(model.argmax_last()[0])
        dec = srq.Decoder(model, cache, first, 63, eager=args.eager)
        ex.synchronize()
        a, b = hip.create(), hip.create()
        hip.record(a, stream)
        dec.run(63)
        hip.record(b, stream)
        times.append(hip.elapsed_ms(a, b))
        tokens = [first] + dec.tokens()
        dec.close()
        cache.close()
    ms = min(times[1:])
    wbytes = synthetic.decode_weight_bytes(cfg, "q8")
    tps = 63 / (ms / 1e3)
    print(json.dumps({
        "metric": "SmolLM2-135M-shape Q8 greedy decode tokens/s, batch 1", "value": round(tps, 1),
        "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "SmolLM2-135M-shape Q8, 32-token random prompt, 64 greedy tokens (63 timed "
                               "graph-replayed decode steps)", "seed": args.seed},
        "ms_per_token": round(ms / 63, 4), "weight_bytes_per_token": wbytes,
        "weight_gbs": round(wbytes * tps / 1e9, 1), "tokens": tokens}), flush=True)
    return 0


def bench_gemv_sweep(srq, args):
    """Isolated Q8 dequant-GEMV at Llama-3.2-1B shapes (hidden 2048,
    intermediate 8192, vocab 128256): weights N(0, 0.02) packed on the
    device, x N(0, 1), batch 1 / 4 / 16, 200 timed launches each (HIP
    events around every launch, on the launch stream): median, p10, p90."""
    ex = srq.Executor(0)
    hip = HipEvents()
    stream = C.c_void_p(ex.stream)
    L = srq.lib()
    shapes = [("q_proj/o_proj", 2048, 2048), ("k_proj/v_proj", 512, 2048), ("gate_proj/up_proj", 8192, 2048),
              ("down_proj", 2048, 8192), ("lm_head", 128256, 2048)]
    out = []
    for t, (name, rows, cols) in enumerate(shapes):
        src = ex.empty(rows * cols * 4)
        srq.fill_normal(ex, src, rows * cols, args.seed * 1000003 + t, 0.02)
        h = C.c_void_p()
        srq.check(L.srq_weight_create(ex.h, srq.Q8, rows, cols, src.ptr, srq.SRC_F32, C.byref(h)))
        w = srq.Weight(h)
        src.close()
        vb, sb = srq.packed_bytes(srq.Q8, rows, cols)
        for n in (1, 4, 16):
            x = ex.empty(n * cols * 4)
            srq.fill_normal(ex, x, n * cols, 7 + n, 1.0)
            y = ex.empty(n * rows * 4)
            for _ in range(10):
                srq.check(L.srq_linear_enqueue(ex.h, y.ptr, x.ptr, w.h, n))
            ex.synchronize()
            evs = [(hip.create(), hip.create()) for _ in range(200)]
            for a, b in evs:
                hip.record(a, stream)
                srq.check(L.srq_linear_enqueue(ex.h, y.ptr, x.ptr, w.h, n))
                hip.record(b, stream)
            ex.synchronize()
            us = [hip.elapsed_ms(a, b) * 1e3 for a, b in evs]
            for a, b in evs:
                hip.destroy(a)
                hip.destroy(b)
            med, p10, p90 = percentiles(us)
            algo = vb + sb + n * cols * 4 + n * rows * 4
            out.append({"matrix": name, "rows": rows, "cols": cols, "n": n, "median_us": round(med, 3),
                        "p10_us": round(p10, 3), "p90_us": round(p90, 3), "algorithmic_bytes": algo,
                        "gbs_median": round(algo / (med * 1e-6) / 1e9, 1),
                        "frac_of_hbm_peak": round(algo / (med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                        "gflops_median": round(2.0 * n * rows * cols / (med * 1e-6) / 1e9, 1)})
            x.close()
            y.close()
        w.close()
    print(json.dumps({"metric": "Q8 dequant-GEMV sweep at Llama-3.2-1B shapes (per launch, HIP events)",
                      "unit": "us", "n_gpus": 1, "higher_is_better": False, "dtype": "f32", "data": "synthetic",
                      "config": {"workload": "Llama-3.2-1B matrices, Q8, batch 1/4/16, 200 launches each",
                                 "seed": args.seed}, "results": out}), flush=True)
    return 0


def bench_q4mixed_prefill(srq, args):
    """Mistral-7B shape, q4-mixed (Q4 layer matrices, Q8 embedding and
    head): a 2048-token random prompt prefilled in 256-token chunks (MFMA
    dequant-GEMM, head only on each chunk's last row), then 128 greedy
    decode tokens."""
    from sr_go_tranformer_amd import synthetic
    ex = srq.Executor(0)
    prompt_n, chunk, gen = args.prompt_tokens, 256, args.gen_tokens
    cfg = synthetic.shape_config("mistral-7b", prompt_n + gen)
    model = synthetic.build(ex, cfg, "q4-mixed", args.seed)
    hip = HipEvents()
    stream = C.c_void_p(ex.stream)
    pool = model.pool((prompt_n + gen) // 32 + 2 + chunk // 32)
    cache = pool.cache((prompt_n + gen + 31) // 32)
    prompt = synthetic.random_prompt(prompt_n, cfg.vocab, args.seed)
    # One untimed chunk on a throwaway cache first, as every other mode warms
    # up: the first 256-row step loads its kernels' code and sizes the step
    # workspace (about 7 ms, once per process).
    warm_cache = pool.cache((chunk + 31) // 32)
    model.step([warm_cache], [prompt[:chunk]])
    warm_cache.close()
    ex.synchronize()
    chunk_ms = []
    for lo in range(0, prompt_n, chunk):
        a, b = hip.create(), hip.create()
        hip.record(a, stream)
        model.step([cache], [prompt[lo:lo + chunk]])
        hip.record(b, stream)
        chunk_ms.append(hip.elapsed_ms(a, b))
    first = int(model.argmax_last()[0])
    dec = srq.Decoder(model, cache, first, gen - 1, eager=args.eager)
    warm = min(4, (gen - 1) // 4)  # untimed decode steps: the decode kernels' first launches
    dec.run(warm)
    ex.synchronize()
    a, b = hip.create(), hip.create()
    hip.record(a, stream)
    dec.run(gen - 1 - warm)
    hip.record(b, stream)
    dec_ms = hip.elapsed_ms(a, b)
    dec.close()
    d, kd, H, V = cfg.dim, cfg.dim // cfg.heads * cfg.kv_heads, cfg.hidden, cfg.vocab
    params = cfg.layers * ((d + 2 * kd) * d + d * d + 2 * H * d + d * H)
    flops_chunk = 2.0 * chunk * params + 2.0 * d * V  # layer GEMMs + one head row
    prefill_s = sum(chunk_ms) / 1e3
    print(json.dumps({
        "metric": "Mistral-7B-shape Q4-mixed chunked prefill tokens/s (256-token chunks) + decode tokens/s",
        "value": round(prompt_n / prefill_s, 1), "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "Mistral-7B shape, q4-mixed, %d random prompt tokens in 256-token chunks, "
                               "then %d greedy tokens" % (prompt_n, gen), "seed": args.seed},
        "chunk_ms": [round(t, 2) for t in chunk_ms],
        "layer_gemm_tflops_per_chunk": round(2.0 * chunk * params / 1e12, 3),
        "achieved_tflops_mean": round(flops_chunk * len(chunk_ms) / prefill_s / 1e12, 2),
        "fp32_mfma_peak_tflops": 157.3,
        "decode_tokens_per_s": round((gen - 1 - warm) / (dec_ms / 1e3), 1),
        "decode_weight_bytes_per_token": synthetic.decode_weight_bytes(cfg, "q4-mixed"),
        "resident_weight_bytes": model.resident_bytes()}), flush=True)
    return 0


def bench_continuous_batching(srq, args):
    """Llama-3.2-3B shape (3072 / 28 layers / 24:8 heads / 8192 / 128256
    tied), Q8, seeded N(0, 0.02) weights: 32 concurrent requests, prompt
    lengths uniform in [64, 1024], 128 output tokens each, paged KV, the
    reference's scheduling defaults (prefill chunk 16, mixed chunk 1, token
    budget 64), sampling at temperature 0.8, top-p 0.9, top-k off, no repeat
    penalty, RNG{seed + i} per request; logits stay on the device."""
    from sr_go_tranformer_amd import synthetic
    from sr_go_tranformer_amd.schedule import TickPlanner
    sessions_n, out_n, budget, chunk, mixed = 32, args.gen_tokens_cb, 64, 16, 1
    r = synthetic.SplitMix64(args.seed)
    lens = [64 + r.intn(1024 - 64 + 1) for _ in range(sessions_n)]
    ex = srq.Executor(0)
    cfg = synthetic.shape_config("llama3.2-3b", max(lens) + out_n + 1)
    model = synthetic.build(ex, cfg, "q8", args.seed)
    prompts = [synthetic.random_prompt(n, cfg.vocab, args.seed * 7 + i) for i, n in enumerate(lens)]
    pages = sum((n + out_n + 31) // 32 for n in lens)
    pool = model.pool(pages + 8)
    caches = [pool.cache((n + out_n + 31) // 32) for n in lens]
    rng = np.array([(args.seed + i) & ((1 << 64) - 1) for i in range(sessions_n)], np.uint64)
    params = srq.Sampling(0.8, 0, 0.9, 1.0)
    tp = TickPlanner(prompts, out_n, budget, chunk, mixed)
    steps, rows_total = 0, 0
    flag = C.c_int32(0) if args.cancel_flag else None  # a context that is never canceled
    ex.synchronize()
    t0 = time.perf_counter()
    while not tp.done():
        sessions, chunks, want = tp.plan()
        dev = model.step([caches[i] for i in sessions], chunks, want=want, host=False, cancel=flag)
        rows_total += sum(len(c) for c in chunks)
        steps += 1
        sel = [k for k in range(len(sessions)) if want[k]]
        sampled = {}
        if sel:
            # the step's logits are [sessions x vocab]; sample the rows of the
            # sessions that asked for a token
            st = rng[[sessions[k] for k in sel]].copy()
            ids = srq.sample(ex, dev, len(sel), cfg.vocab, params, st, row_ids=sel)
            for j, k in enumerate(sel):
                rng[sessions[k]] = st[j]
                sampled[sessions[k]] = int(ids[j])
        live = set(tp.live)
        tp.commit(sampled)
        for i in live - set(tp.live):
            caches[i].close()
    ex.synchronize()
    dt = time.perf_counter() - t0
    gen = sum(len(o) for o in tp.outputs)
    print(json.dumps({
        "metric": "Llama-3.2-3B-shape Q8 continuous batching output tokens/s (32 requests)",
        "value": round(gen / dt, 1), "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "Llama-3.2-3B shape, Q8, 32 requests, prompts U[64,1024], %d outputs each, "
                               "budget 64 / chunk 16 / mixed 1, T 0.8 top-p 0.9" % out_n, "seed": args.seed,
                   "cancel_flag": bool(args.cancel_flag)},
        "seconds": round(dt, 3), "steps": steps, "rows_processed": rows_total,
        "rows_per_s": round(rows_total / dt, 1), "ms_per_step": round(dt * 1e3 / steps, 3),
        "prompt_tokens": sum(lens), "generated_tokens": gen}), flush=True)
    return 0


def bench_step_decode(srq, args):
    """Mistral-7B shape, Q8, batch 1: the 128-token prompt prefilled in one
    step, then greedy decode one srq_step per token (logits on the device,
    device argmax), as an engine drives it without the graph decoder;
    --cancel-flag passes a flag that is never raised, so the step paces its
    layers for cancellation."""
    from sr_go_tranformer_amd import synthetic
    ex = srq.Executor(0)
    cfg = synthetic.shape_config("mistral-7b", PROMPT + args.warmup + args.steps + 2)
    model = synthetic.build(ex, cfg, "q8", args.seed)
    prompt = synthetic.random_prompt(PROMPT, cfg.vocab, args.seed)
    pool = model.pool((PROMPT + args.warmup + args.steps + 2) // 32 + 2)
    cache = pool.cache((PROMPT + args.warmup + args.steps + 2) // 32 + 1)
    flag = C.c_int32(0) if args.cancel_flag else None
    model.step([cache], [prompt], host=False, cancel=flag)
    tok = int(model.argmax_last()[0])
    for _ in range(args.warmup):
        model.step([cache], [[tok]], host=False, cancel=flag)
        tok = int(model.argmax_last()[0])
    ex.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.step([cache], [[tok]], host=False, cancel=flag)
        tok = int(model.argmax_last()[0])
    ex.synchronize()
    dt = time.perf_counter() - t0
    print(json.dumps({
        "metric": "Mistral-7B-shape Q8 decode tokens/s, one srq_step per token", "value": round(args.steps / dt, 2),
        "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "Mistral-7B shape, Q8, batch 1, 128-token prompt, %d untimed and %d timed greedy "
                               "decode steps through srq_step + srq_argmax" % (args.warmup, args.steps),
                   "seed": args.seed, "cancel_flag": bool(args.cancel_flag)},
        "ms_per_step": round(dt * 1e3 / args.steps, 4)}), flush=True)
    return 0


def bench_longctx_decode(srq, args):
    """Mistral-7B shape, Q8: a long random prompt (default 8192 tokens)
    prefilled in 256-token chunks, then greedy decode at that context.  The
    paged KV cache then holds 2*ctx*kv_dim*4 bytes per layer, which every
    decode token reads: at 8k context, 2.1 GB next to 7.6 GB of weights."""
    from sr_go_tranformer_amd import synthetic
    ex = srq.Executor(0)
    prompt_n, chunk, gen = args.context_tokens, 256, args.gen_tokens
    cfg = synthetic.shape_config("mistral-7b", prompt_n + gen)
    model = synthetic.build(ex, cfg, "q8", args.seed)
    hip = HipEvents()
    stream = C.c_void_p(ex.stream)
    pool = model.pool((prompt_n + gen) // 32 + 2 + chunk // 32)
    cache = pool.cache((prompt_n + gen + 31) // 32)
    prompt = synthetic.random_prompt(prompt_n, cfg.vocab, args.seed)
    warm_cache = pool.cache((chunk + 31) // 32)  # one untimed chunk, as in the prefill bench
    model.step([warm_cache], [prompt[:chunk]])
    warm_cache.close()
    ex.synchronize()
    a, b = hip.create(), hip.create()
    hip.record(a, stream)
    for lo in range(0, prompt_n, chunk):
        model.step([cache], [prompt[lo:lo + chunk]])
    hip.record(b, stream)
    prefill_ms = hip.elapsed_ms(a, b)
    first = int(model.argmax_last()[0])
    dec = srq.Decoder(model, cache, first, gen - 1, eager=args.eager)
    warm = min(4, (gen - 1) // 4)  # untimed decode steps: the decode kernels' first launches
    dec.run(warm)
    ex.synchronize()
    hip.record(a, stream)
    dec.run(gen - 1 - warm)
    hip.record(b, stream)
    dec_ms = hip.elapsed_ms(a, b)
    dec.close()
    kd = cfg.dim // cfg.heads * cfg.kv_heads
    wbytes = synthetic.decode_weight_bytes(cfg, "q8")
    mid = prompt_n + gen // 2
    kv_bytes = 2 * mid * kd * 4 * cfg.layers
    tok_s = (gen - 1 - warm) / (dec_ms / 1e3)
    print(json.dumps({
        "metric": "Mistral-7B-shape Q8 long-context greedy decode tokens/s (paged KV)",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "Mistral-7B shape, Q8, %d random prompt tokens in 256-token chunks, then %d greedy "
                               "tokens" % (prompt_n, gen), "seed": args.seed,
                   "decode_launch": "eager" if args.eager else "hip-graph"},
        "prefill_tokens_per_s": round(prompt_n / (prefill_ms / 1e3), 1),
        "decode_ms_per_token": round(dec_ms / (gen - 1 - warm), 4),
        "weight_bytes_per_token": wbytes, "kv_bytes_per_token_mid": kv_bytes,
        "achieved_gb_per_s": round((wbytes + kv_bytes) * tok_s / 1e9, 1),
        "frac_of_hbm_peak": round((wbytes + kv_bytes) * tok_s / 8e12, 4)}), flush=True)
    return 0


def write_bf16_archive(directory, cfg, seed, shard_bytes=5 << 30):
    """A Transformers directory of the given config.json dict whose tensors
    are BF16 words of N(0, 0.02) values (a 32 Mi-word block repeated), in
    shards of at most shard_bytes with an index.  Returns the archive size."""
    rng = np.random.default_rng(seed)
    block = (rng.normal(0.0, 0.02, 16 << 20).astype(np.float32).view(np.uint32) >> 16).astype("<u2").tobytes()
    d, h, v, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"], cfg["num_hidden_layers"]
    kd = d // cfg["num_attention_heads"] * cfg["num_key_value_heads"]
    specs = [("model.embed_tokens.weight", [v, d])]
    for i in range(L):
        p = "model.layers.%d." % i
        specs += [(p + "input_layernorm.weight", [d]), (p + "self_attn.q_proj.weight", [d, d]),
                  (p + "self_attn.k_proj.weight", [kd, d]), (p + "self_attn.v_proj.weight", [kd, d]),
                  (p + "self_attn.o_proj.weight", [d, d]), (p + "post_attention_layernorm.weight", [d]),
                  (p + "mlp.gate_proj.weight", [h, d]), (p + "mlp.up_proj.weight", [h, d]),
                  (p + "mlp.down_proj.weight", [d, h])]
    specs += [("model.norm.weight", [d]), ("lm_head.weight", [v, d])]
    groups, cur, size = [], [], 0
    for name, shape in specs:
        n = 2 * int(np.prod(shape))
        if cur and size + n > shard_bytes:
            groups.append(cur)
            cur, size = [], 0
        cur.append((name, shape, n))
        size += n
    groups.append(cur)
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(cfg, f)
    index, total = {}, 0
    for i, group in enumerate(groups):
        fname = "model-%05d-of-%05d.safetensors" % (i + 1, len(groups))
        header, off = {}, 0
        for name, shape, n in group:
            header[name] = {"dtype": "BF16", "shape": shape, "data_offsets": [off, off + n]}
            off += n
            index[name] = fname
        hb = json.dumps(header).encode()
        with open(os.path.join(directory, fname), "wb") as f:
            f.write(len(hb).to_bytes(8, "little") + hb)
            left = off
            while left > 0:
                k = min(left, len(block))
                f.write(block[:k])
                left -= k
        total += 8 + len(hb) + off
        print("archive shard %d/%d written" % (i + 1, len(groups)), file=sys.stderr, flush=True)
    with open(os.path.join(directory, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": index}, f)
    return total


def bench_archive_load(srq, args):
    """Load a Mistral-7B-shape BF16 Transformers archive (three ~5 GB shards
    in the page cache) into a Q8 model: archive checks, pread into pinned
    slots, copies and device packing (srq_model_load_safetensors)."""
    import shutil
    import tempfile
    from sr_go_tranformer_amd import hf
    cfg = {"architectures": ["MistralForCausalLM"], "model_type": "mistral", "vocab_size": 32768,
           "hidden_size": 4096, "intermediate_size": 14336, "num_hidden_layers": 32, "num_attention_heads": 32,
           "num_key_value_heads": 8, "max_position_embeddings": 32768, "rope_theta": 1000000.0,
           "rms_norm_eps": 1e-5, "hidden_act": "silu", "tie_word_embeddings": False, "bos_token_id": 1,
           "eos_token_id": 2, "sliding_window": None}
    root = tempfile.mkdtemp(prefix="srq_archive_", dir=args.archive_dir)
    try:
        if shutil.disk_usage(root).free < 20e9:
            print("need 20 GB free under %s for the archive" % root, file=sys.stderr)
            return 2
        size = write_bf16_archive(root, cfg, args.seed)
        ex = srq.Executor(0)
        times = []
        for _ in range(3):
            m, _ = hf.open_model(ex, root, "q8", context_limit=4096)
            ex.synchronize()
            m.close()
            t0 = time.perf_counter()
            m, _ = hf.open_model(ex, root, "q8", context_limit=4096)
            ex.synchronize()
            times.append(time.perf_counter() - t0)
            m.close()
        ex.close()
    finally:
        shutil.rmtree(root, ignore_errors=True)
    best = min(times)
    print(json.dumps({
        "metric": "Mistral-7B-shape BF16 safetensors archive load to Q8 (GB/s of archive)",
        "value": round(size / best / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "bf16->q8", "data": "synthetic",
        "config": {"workload": "Mistral-7B shape, 3 BF16 shards in the page cache, config.json read, archive "
                               "checked, loaded and packed to Q8", "archive_bytes": size, "seed": args.seed},
        "seconds": [round(t, 3) for t in times]}), flush=True)
    return 0


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=15, help="untimed decode tokens")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--cpu-tokens", type=int, default=32, help="decode tokens of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--gemv-launches", type=int, default=320)
    ap.add_argument("--config", default="mistral7b-q8-decode",
                    choices=["mistral7b-q8-decode", "mistral7b-q4mixed-decode", "smollm2-q8-decode",
                             "llama1b-q8-gemv-sweep",
                             "mistral7b-q4mixed-prefill", "llama3b-q8-continuous-batching",
                             "mistral7b-q8-longctx-decode", "mistral7b-bf16-archive-load",
                             "mistral7b-q8-step-decode"],
                    help="workload; the default is the headline Mistral-7B Q8 decode")
    ap.add_argument("--prompt-tokens", type=int, default=2048, help="mistral7b-q4mixed-prefill: prompt length")
    ap.add_argument("--gen-tokens", type=int, default=128,
                    help="mistral7b-q4mixed-prefill / mistral7b-q8-longctx-decode: generated tokens")
    ap.add_argument("--context-tokens", type=int, default=8192, help="mistral7b-q8-longctx-decode: prompt length")
    ap.add_argument("--gen-tokens-cb", type=int, default=128,
                    help="llama3b-q8-continuous-batching: output tokens per request")
    ap.add_argument("--gemv-only", action="store_true",
                    help="run only the GEMV roofline leg (standalone weights) and a calibration copy")
    ap.add_argument("--gemv-rows", type=int, default=28672, help="--gemv-only: weight rows (4096 columns)")
    ap.add_argument("--gemv-fmt", default="q8", choices=["q8", "q4"], help="--gemv-only: weight format")
    ap.add_argument("--archive-dir", default=None,
                    help="mistral7b-bf16-archive-load: where the temporary archive is written (default: TMPDIR)")
    ap.add_argument("--cancel-flag", action="store_true",
                    help="llama3b-q8-continuous-batching / mistral7b-q8-step-decode: pass every srq_step a "
                         "cancel flag that stays 0 (the step then paces its layers for cancellation)")
    ap.add_argument("--eager", action="store_true",
                    help="launch each decode kernel directly instead of replaying the captured graph "
                         "(for kernel tracers that cannot follow graph launches)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (--gpus must be 1).", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0 or args.steps + args.warmup > TOKENS - 1:
        print("need 1 <= steps and steps + warmup <= %d (a %d-token generation)" % (TOKENS - 1, TOKENS),
              file=sys.stderr)
        return 2

    import sr_go_tranformer_amd as srq
    from sr_go_tranformer_amd import synthetic

    if args.gemv_only:
        return gemv_only(srq, args.gemv_launches, args.seed, args.gemv_rows, args.gemv_fmt)
    if args.config == "smollm2-q8-decode":
        return bench_smollm2(srq, args)
    if args.config == "llama1b-q8-gemv-sweep":
        return bench_gemv_sweep(srq, args)
    if args.config == "mistral7b-q4mixed-prefill":
        return bench_q4mixed_prefill(srq, args)
    if args.config == "llama3b-q8-continuous-batching":
        return bench_continuous_batching(srq, args)
    if args.config == "mistral7b-q8-step-decode":
        return bench_step_decode(srq, args)
    if args.config == "mistral7b-q8-longctx-decode":
        return bench_longctx_decode(srq, args)
    if args.config == "mistral7b-bf16-archive-load":
        return bench_archive_load(srq, args)

    fmt = "q4-mixed" if args.config == "mistral7b-q4mixed-decode" else "q8"
    t_start = time.perf_counter()
    ex = srq.Executor(0)
    cfg = synthetic.shape_config("mistral-7b", PROMPT + TOKENS)
    model = synthetic.build(ex, cfg, fmt, args.seed)
    build_s = time.perf_counter() - t_start
    resident = model.resident_bytes()
    print("model built in %.1f s, resident %d bytes" % (build_s, resident), file=sys.stderr, flush=True)

    hip = HipEvents()
    stream = C.c_void_p(ex.stream)
    warm_pages = (PROMPT + 31) // 32
    pool = model.pool(16 + warm_pages)
    cache = pool.cache((PROMPT + TOKENS + 31) // 32)
    prompt = synthetic.random_prompt(PROMPT, cfg.vocab, args.seed)
    # One untimed prefill on a throwaway cache first, as the other modes warm
    # up: a process's first step loads its kernels' code and sizes the step
    # workspace, which is not prefill work.
    warm_cache = pool.cache(warm_pages)
    model.step([warm_cache], [prompt])
    warm_cache.close()
    ex.synchronize()
    t0 = time.perf_counter()
    model.step([cache], [prompt])
    prefill_s = time.perf_counter() - t0
    first = int(model.argmax_last()[0])

    dec = srq.Decoder(model, cache, first, args.warmup + args.steps, eager=args.eager)
    dec.run(args.warmup)
    ex.synchronize()
    ev0, ev1 = hip.create(), hip.create()
    hip.record(ev0, stream)
    dec.run(args.steps)
    hip.record(ev1, stream)
    ex.synchronize()
    decode_ms = hip.elapsed_ms(ev0, ev1)
    tokens = dec.tokens()
    dec.close()
    print("decode %d tokens in %.2f ms" % (args.steps, decode_ms), file=sys.stderr, flush=True)

    ms_per_step = decode_ms / args.steps
    tok_s = 1e3 / ms_per_step
    wbytes = synthetic.decode_weight_bytes(cfg, fmt)
    gbs = wbytes * tok_s / 1e9
    kd = cfg.dim // cfg.heads * cfg.kv_heads
    pos_mid = PROMPT + args.warmup + args.steps / 2.0
    kv_bytes = 2 * pos_mid * kd * 4 * cfg.layers

    # The decode step's dominant kernel streams the fused gate/up matrix
    # (28672 x 4096 per layer); the 14336 x 4096 up projection alone is the
    # shape the reference's published GEMV table quotes.
    gus = [model.weight(srq.T_GATE_UP, layer) for layer in range(cfg.layers)]
    roof = gemv_roofline(srq, ex, gus, hip, args.gemv_launches,
                         "the fused gate/up storage of the 32 layers, the decode step's dominant matrix")
    ups = [model.weight(srq.T_UP, layer) for layer in range(cfg.layers)]
    roof_up = gemv_roofline(srq, ex, ups, hip, args.gemv_launches, "the up projection alone, 32 layers")
    print("gemv %.1f GB/s (gate/up), %.1f GB/s (up)" % (roof["achieved"], roof_up["achieved"]), file=sys.stderr,
          flush=True)

    cpu = None
    if fmt != "q8":
        tag = "Q4" if fmt == "q4-mixed" else fmt
        out = {
            "metric": "Mistral-7B-shape %s decode tokens/s and weight GB/s, batch 1" % fmt,
            "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "Mistral-7B shape, %s (layer matrices %s, embedding and head Q8), 128-token "
                                   "random prompt, %d greedy tokens (%d untimed, %d timed graph-replayed steps)" %
                                   (fmt, tag, 1 + args.warmup + args.steps, args.warmup, args.steps),
                       "seed": args.seed, "decode_launch": "eager" if args.eager else "hip-graph"},
            "weight_bytes_per_token": wbytes, "weight_gb_per_s": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "resident_weight_bytes": resident,
            "roofline": roof, "gemv_14336x4096": {k: roof_up[k] for k in ("kernel", "achieved", "frac", "traffic",
                                                                           "avg_launch_us")}}
        print(json.dumps(out), flush=True)
        return 0
    if not args.no_cpu_baseline:
        # the oracle decodes the GPU's own token sequence (first + replays)
        n = max(1, min(args.cpu_tokens, len(tokens)))
        runs, setup_s = cpu_baseline(srq, ex, model, cfg, cache, first, tokens, n)
        (workers, tps, produced), (w4, tps4, produced4) = runs
        host = host_facts()
        cpu = {"value": round(wbytes * tps / 1e9, 3), "unit": "GB/s", "tokens_per_s": round(tps, 4),
               "cores": workers, "kind": "port",
               "sample": "%d greedy decode tokens of the same Mistral-7B-shape Q8 model from position %d "
                         "(KV rows copied from the GPU prefill), oracle C restatement of the reference Go "
                         "CPU path, %d worker threads (GOMAXPROCS-equivalent) on a %d-CPU host (%s)" %
                         (n, PROMPT, workers, host["nproc"], host["cpu_model"]),
               "nproc": host["nproc"], "cpu_model": host["cpu_model"], "gomaxprocs_equivalent": workers,
               "greedy_match": produced == tokens[:len(produced)],
               "threads_4": {"value": round(wbytes * tps4 / 1e9, 3), "tokens_per_s": round(tps4, 4),
                             "tokens": len(produced4), "gomaxprocs_equivalent": 4,
                             "greedy_match": produced4 == tokens[:len(produced4)]}}
        print("cpu %.3f tok/s (%d threads), %.3f tok/s (4 threads)" % (tps, workers, tps4), file=sys.stderr,
              flush=True)

    out = {
        "metric": "Q8 decode GEMV HBM GB/s (% of peak) + tokens/s, 7B-shape, batch 1",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(gbs / REF_GBS, 1),
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "Mistral-7B-shape Q8 greedy decode, batch 1, 128-token random prompt, %d greedy tokens "
                        "(the first from the prefill, %d untimed and %d timed graph-replayed decode steps)" %
                        (1 + args.warmup + args.steps, args.warmup, args.steps),
            "hidden": cfg.dim, "layers": cfg.layers, "heads": cfg.heads, "kv_heads": cfg.kv_heads,
            "intermediate": cfg.hidden, "vocab": cfg.vocab, "page_tokens": 32, "weights": "int8 Q8, f32 scales/64",
            "prompt_tokens": PROMPT, "generated_tokens": 1 + args.warmup + args.steps, "timed_tokens": args.steps,
            "seed": args.seed,
            "decode_launch": "eager" if args.eager else "hip-graph",
            "vs_baseline_reference": "Mistral-7B Q8 decode batch 1 on Apple M4 (GOMAXPROCS=4): 1.33 tok/s, "
                                     "10.1 GB/s of weights",
        },
        "tokens_per_s": round(tok_s, 2),
        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "weight_bytes_per_token": wbytes,
        "kv_bytes_per_token_mid": int(kv_bytes),
        "prefill_tokens_per_s": round(PROMPT / prefill_s, 1),
        "resident_weight_bytes": resident,
        "roofline": roof,
        "gemv_14336x4096": {k: roof_up[k] for k in ("kernel", "achieved", "frac", "traffic", "avg_launch_us")},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
