#!/usr/bin/env python3
"""MoE-stack decode benchmark on one MI355X.

Headline workload: the MoE half of one GLM-4.7-Flash decode step -- 46 MoE layers in
sequence (hidden 2048, 64 routed experts + 1 shared, moe_intermediate 1536, top-4,
Q8_0 experts), T=1, per-layer seeded synthetic weights resident in HBM (~30 GB),
RMSNorm inside every layer (infer.c:1098). A step is one token through all 46 layers
via gmoe_forward_layers; every step starts from the same input.

Prints one JSON line: tokens/s (value), the per-layer time and the HBM rate on the
selected experts' Q8_0 bytes, the roofline of the dominant kernel (its HIP-event launch
time against MI355X's 8 TB/s) and the reference CPU path timed on this host (glm.c's
own infer.c built from source, OpenMP bound to cores as glm.c's Makefile runs it, same
weights). Extra keys time the other workloads on the same resident layers: one MoE
layer per launch (rotating over the 46), prefill batches of T=512 (near-uniform
routing) and T=128 (Zipf(1.2)-skewed routing) on the grouped expert GEMMs, the
glm.c drop-in hook (glm_backend_try_hip_moe on a RunState in host memory), the decode step
and a T=512 prefill layer on layers in glm.c's exported form (group size 16, fp32 scales),
and the whole GLM-4.7-Flash-shaped model on the GPU: a 4096-token prompt by batched
prefill, then 128 tokens decoded one at a time.
"""
import os

# glm.c's Makefile runs the CPU path with threads bound to cores (Makefile:89-92). libgomp
# reads these when it loads, so they are set before anything loads it.
os.environ.setdefault("OMP_PROC_BIND", "true")
os.environ.setdefault("OMP_PLACES", "cores")
# the CPUs this process may use, read before libgomp binds the initial thread to one of them
CPUS_ALLOWED = len(os.sched_getaffinity(0))

import argparse  # noqa: E402
import json  # noqa: E402
import subprocess  # noqa: E402
import sys  # noqa: E402
import time  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "glm.c_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16
N_MOE_LAYERS = 46
PREFILL_BATCH = 1024  # prompt tokens per batched prefill step of the end-to-end run
METRIC = "MoE-stack decode tokens/s (46 GLM-4.7-Flash MoE layers, Q8_0, T=1)"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def omp_threads():
    import ctypes
    try:
        gomp = ctypes.CDLL("libgomp.so.1")
        return int(gomp.omp_get_max_threads())
    except OSError:
        return int(os.environ.get("OMP_NUM_THREADS", "1"))


def host_cpus():
    """Physical cores of this host (lscpu: cores per socket x sockets) and the CPUs this
    process may run on."""
    phys = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = dict(line.split(":", 1) for line in out.splitlines() if ":" in line)
        phys = int(kv["Core(s) per socket"].strip()) * int(kv["Socket(s)"].strip())
    except (OSError, KeyError, ValueError, subprocess.SubprocessError):
        pass
    return {"host_physical_cores": phys, "cpus_allowed": CPUS_ALLOWED,
            "omp_proc_bind": os.environ.get("OMP_PROC_BIND"), "omp_places": os.environ.get("OMP_PLACES")}


def traffic_from_profiles(kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summary, or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return t[kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def median(v):
    v = sorted(v)
    return v[len(v) // 2]


def latency_stats(ms):
    """Per-token latencies as glm.c's bench mode reports them (infer.c:1452-1462,
    1564-1581): the mean, and p50 and p95 interpolated linearly between the sorted times
    at rank q/100 * (n - 1)."""
    v = sorted(ms)
    n = len(v)

    def pct(q):
        r = q / 100.0 * (n - 1)
        lo = int(r)
        if lo + 1 >= n:
            return v[-1]
        return v[lo] * (1.0 - (r - lo)) + v[lo + 1] * (r - lo)

    return {"tokens": n, "mean_ms": round(sum(v) / n, 4), "p50_ms": round(pct(50), 4), "p95_ms": round(pct(95), 4),
            "min_ms": round(v[0], 4), "max_ms": round(v[-1], 4)}


def cpu_baseline(shape, host_layers, x0, seconds):
    """glm.c's CPU MoE path (infer.c, OpenMP) on the same layers: decode tokens through the
    46-layer stack, every layer call timed with glm.c's monotonic clock (infer.c:1426-1430).
    All of the process's threads (OMP_NUM_THREADS) for about `seconds`, then one thread
    for two tokens."""
    import numpy as np
    import oracle

    if not oracle.available("reference"):
        return None
    threads = omp_threads()
    oracle.stack_timed(shape, host_layers, x0, 1, threads)  # warm the page cache and the thread pool
    ms = oracle.stack_timed(shape, host_layers, x0, 1, threads)
    n_tok = max(20, int(seconds * 1e3 / max(1e-3, float(ms.sum()))))
    ms = oracle.stack_timed(shape, host_layers, x0, n_tok, threads)
    tok_ms = median(ms.sum(axis=1).tolist())
    one = oracle.stack_timed(shape, host_layers, x0, 2, 1)
    oracle.stack_timed(shape, host_layers[:1], x0, 1, threads)  # back to the full team
    per_layer_bytes = (shape.K + 1) * shape.expert_bytes()
    layer_ms = median(ms.ravel().tolist())
    return {
        "value": round(1e3 / tok_ms, 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "reference",
        "sample": f"{n_tok} decode tokens through the same {len(host_layers)}-layer stack (glm.c's infer.c built "
                  f"with its Makefile flags, OpenMP threads bound to cores), median per-token time; "
                  f"{n_tok * len(host_layers)} timed layer calls",
        "ms_per_token": round(tok_ms, 3),
        "layer_us": round(layer_ms * 1e3, 1),
        "layer_gbs_expert_bytes": round(per_layer_bytes / (layer_ms * 1e-3) / 1e9, 2),
        "one_thread": {"tokens_s": round(1e3 / median(one.sum(axis=1).tolist()), 3),
                       "layer_us": round(median(one.ravel().tolist()) * 1e3, 1),
                       "sample": f"2 tokens x {len(host_layers)} layers, one OpenMP thread"},
        **host_cpus(),
    }


def cpu_prefill_baseline(shape, host_layer, x, n_calls=24):
    """glm.c's prefill is one decode call per prompt token (infer.c:2190-2233): the median
    of n_calls timed single-token layer calls on tokens of the same batch."""
    import oracle

    if not oracle.available("reference"):
        return None
    threads = omp_threads()
    oracle.layer_timed(shape, host_layer, x[:2], threads)
    ms = oracle.layer_timed(shape, host_layer, x[:n_calls], threads)
    med = median(ms.tolist())
    return {"value": round(1e3 / med, 2), "unit": "tokens/s", "cores": threads, "kind": "reference",
            "sample": f"median of {n_calls} single-token layer calls (glm.c routes prefill tokens one at a time)",
            "token_us": round(med * 1e3, 1)}


def hip_events_us(gmoe, stream, fn, n):
    """Average µs per call of fn() over n calls, from HIP events on `stream`."""
    a, b = gmoe.Event(), gmoe.Event()
    a.record(stream)
    for _ in range(n):
        fn()
    b.record(stream)
    return a.elapsed_ms(b) * 1e3 / n


def time_prefill(gmoe, np, ctx, shape, layer_ids, T, x, warmup, steps, profile_steps):
    """One layer over T tokens per launch sequence, rotating over layer_ids (so no layer's
    touched experts are still cached from the step before). Returns a result dict."""
    d_in = gmoe.DeviceArray.from_numpy(x)
    d_out = gmoe.DeviceArray(x.nbytes)
    stream = gmoe.Stream()
    it = [0]

    def step():
        ctx.forward(layer_ids[it[0] % len(layer_ids)], T, d_in.ptr, d_out.ptr, stream=stream.h)
        it[0] += 1

    for _ in range(warmup):
        step()
    stream.sync()
    t_begin = time.perf_counter()
    for _ in range(steps):
        step()
    stream.sync()
    layer_us = (time.perf_counter() - t_begin) * 1e6 / steps
    touched, pairs = [], []
    for layer in layer_ids:
        _, st = gmoe.forward_host(ctx, layer, x)
        counts = np.diff(st["expert_offsets"])
        touched.append(int(np.sum(counts > 0)) + 1)
        pairs.append(int(counts.sum()) + T)
    bytes_per_layer = float(np.mean(touched)) * shape.expert_bytes()
    macs = float(np.mean(pairs)) * 3 * shape.F * shape.D
    ctx.profile(True)
    for _ in range(profile_steps):
        step()
    stream.sync()
    prof = ctx.profile_read()
    ctx.profile(False)
    kernels = {k: {"launches": n, "avg_us": round(ms * 1e3 / n, 3)} for k, (n, ms) in prof.items()}
    gemm_us = sum(kernels[k]["avg_us"] for k in ("gate_up", "down") if k in kernels)
    tflops = 2.0 * macs / (gemm_us * 1e-6) / 1e12 if gemm_us else 0.0
    gbs = bytes_per_layer / (layer_us * 1e-6) / 1e9
    return {
        "tokens_s": round(T / (layer_us * 1e-6), 1),
        "layer_us": round(layer_us, 2),
        "touched_experts": round(float(np.mean(touched)), 2),
        "hbm_gbps_touched_bytes": round(gbs, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "mfma": {"algorithmic_tflops": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                 "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                 "note": "algorithmic 2*MACs of the expert products over the two grouped GEMM kernels' time; the "
                         "kernels execute 2x those MACs (hi and lo planes) plus tile padding"},
        "kernels": kernels,
    }


def gs16_form(gmoe, np, args, L):
    """glm.c's exported checkpoint form (group size 16, fp32 scales, glm47_flash_export.py:36,
    157-169) on the fast path: the same 46-layer decode step and a T=512 prefill layer,
    seeded layers of that form uploaded to a second context (GMOE_Q8_TILED16)."""
    shape = gmoe.Shape(group_size=16)
    ctx = gmoe.Context(shape, n_layers=L + 1, max_tokens=512, device=0)
    try:
        t0 = time.perf_counter()
        for layer in range(1, L + 1):
            ctx.upload(layer, gmoe.HostLayer(shape, seed=0, layer=layer, scale_mode=gmoe.SYNTH_SCALES_FP32))
        log(f"gs16: generated and uploaded {L} layers in {time.perf_counter() - t0:.1f}s")
        x0 = gmoe.activations(0, 0, 1, shape.D)
        d_in = gmoe.DeviceArray.from_numpy(x0)
        d_out = gmoe.DeviceArray(x0.nbytes)
        stream = gmoe.Stream()

        def step():
            ctx.forward_layers(1, L, 1, d_in.ptr, d_out.ptr, stream=stream.h)

        for _ in range(args.warmup):
            step()
        stream.sync()
        t_begin = time.perf_counter()
        for _ in range(args.steps):
            step()
        stream.sync()
        ms = (time.perf_counter() - t_begin) * 1e3 / args.steps
        stats = ctx.stats()
        bpt = 0
        for layer in range(1, L + 1):
            idx, _ = ctx.read_topk(layer, 1)
            bpt += (int(np.sum(idx >= 0)) + 1) * shape.expert_bytes()
        ctx.profile(True)
        for _ in range(max(1, args.profile_steps // 5)):
            step()
        stream.sync()
        prof = ctx.profile_read()
        ctx.profile(False)
        kern = {k: {"launches": n, "avg_us": round(t * 1e3 / n, 3)} for k, (n, t) in prof.items()}
        gbs = bpt / (ms * 1e-3) / 1e9
        out = {"workload": "46 GLM-4.7-Flash MoE layers, T=1, group size 16 with fp32 scales (the exporter's form)",
               "q8_form": "tiled16" if stats["q8_form"] == gmoe.GMOE_Q8_TILED16 else str(stats["q8_form"]),
               "decode_tokens_s": round(1e3 / ms, 2), "layer_us": round(ms * 1e3 / L, 3),
               "expert_bytes_per_token": bpt, "hbm_gbps_expert_bytes": round(gbs, 1),
               "hbm_frac_expert_bytes": round(gbs / HBM_PEAK_GBS, 4), "kernels": kern}
        NL = min(args.prefill_layers, L)
        x512 = gmoe.activations(0, 1, 512, shape.D)
        out["prefill_t512"] = time_prefill(gmoe, np, ctx, shape, list(range(1, NL + 1)), 512, x512,
                                           max(2, args.warmup), max(10, args.steps), 10)
        return out
    finally:
        ctx.close()


def gs16_only(args, gmoe, np):
    """--group-size 16 without --prefill: the exporter's form alone (gs16_form), one JSON line."""
    if gmoe.device_count() < 1:
        raise SystemExit("no HIP device visible")
    res = gs16_form(gmoe, np, args, args.layers)
    out = {
        "metric": "MoE-stack decode tokens/s (46 GLM-4.7-Flash MoE layers, Q8_0 at group size 16 with fp32 scales, T=1)",
        "value": res["decode_tokens_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 / res["decode_tokens_s"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint8->int32 + fp32",
        "data": "synthetic (seeded random-init Q8_0 weights, fp32 scales, N(0,1) input)",
        "config": {"workload": res["workload"], "layers": args.layers},
        **{k: v for k, v in res.items() if k not in ("workload", "decode_tokens_s")},
    }
    print(json.dumps(out), flush=True)


def backend_hook_us(gmoe, np, shape, host_layers, x0, tokens=2):
    """glm.c's drop-in path: glm_backend_init(BACKEND_HIP) uploads the layers, then
    glm_backend_try_hip_moe runs each MoE layer on a RunState in host memory (an H2D copy of
    x, the layer, a synchronisation and the D2H copies of x and the intermediates glm.c
    keeps in its RunState). Median µs per layer call over `tokens` decode tokens."""
    import glm_model

    model = glm_model.GlmModel(shape, host_layers)
    if model.init() != glm_model.BACKEND_HIP:
        raise SystemExit("glm_backend_init(BACKEND_HIP) did not select the HIP backend")
    try:
        model.buf["x"][:] = x0[0]
        for layer in range(1, len(host_layers) + 1):  # warm-up token
            if model.try_moe(layer) != 0:
                raise SystemExit(f"glm_backend_try_hip_moe declined layer {layer}")
        times = []
        for _ in range(tokens):
            for layer in range(1, len(host_layers) + 1):
                t0 = time.perf_counter()
                rc = model.try_moe(layer)
                times.append(time.perf_counter() - t0)
                if rc != 0:
                    raise SystemExit(f"glm_backend_try_hip_moe declined layer {layer}")
    finally:
        model.free()
    return {"layer_us": round(median(times) * 1e6, 2), "calls": len(times),
            "note": "per-layer wall time of glm_backend_try_hip_moe, host RunState in and out (PCIe-inclusive)"}


def e2e_decode(gmoe, np, ctx, context=4096, new=128, seed=0):
    """The whole GLM-4.7-Flash-shaped model on the GPU (gmoe_model): random-init dense side
    (47 layers of MLA attention, dense layer 0, vocabulary 154880, all Q8_0) around the MoE
    layers 1..46 already resident in ctx. A `context`-token prompt goes in by batched
    prefill, then `new` tokens are decoded one at a time, each picked greedily on the host
    from the logits of the step before (as glm.c's loop samples, infer.c:2190-2231)."""
    cfg = dict(gmoe.GLM47_FLASH_MODEL, cache_cap=context + new, attn_layers=47, has_l0_ffn=1, max_batch=ctx.max_tokens)
    t0 = time.perf_counter()
    g, layers = gmoe.synth_model_weights(cfg, seed)
    model = gmoe.Model(cfg)
    try:
        model.upload(g)
        for l, a in enumerate(layers):
            model.upload_attn(l, a)
        del g, layers
        model.set_moe(ctx, range(1, cfg["n_layers"]))
        log(f"e2e model: dense side generated and uploaded in {time.perf_counter() - t0:.1f}s")
        rng = np.random.default_rng(seed)
        prompt = rng.integers(3, cfg["vocab_size"], context).astype(np.int32)
        B = ctx.max_tokens
        model.prefill(prompt[:B], 0)  # warm-up, rewritten below
        t0 = time.perf_counter()
        for i in range(0, context, B):
            logits = model.prefill(prompt[i:i + B], i)
        prefill_s = time.perf_counter() - t0
        tok = int(np.argmax(logits))
        for _ in range(2):  # warm-up steps that leave the cache as it was
            model.forward_token(tok, context, flags=1)
        t0 = time.perf_counter()
        tok_ms = []
        for i in range(new):
            t1 = time.perf_counter()
            tok = int(np.argmax(model.forward_token(tok, context + i)))
            tok_ms.append((time.perf_counter() - t1) * 1e3)
        decode_s = time.perf_counter() - t0
    finally:
        model.close()
    return {"workload": f"GLM-4.7-Flash-shaped model (47 layers, vocab {cfg['vocab_size']}), {new} new tokens "
                        f"decoded greedily after a {context}-token prompt; random-init Q8_0 weights",
            "decode_tokens_s": round(new / decode_s, 2), "decode_ms_per_token": round(decode_s * 1e3 / new, 3),
            "decode_per_token": latency_stats(tok_ms),
            "prefill_tokens_s": round(context / prefill_s, 1), "prefill_batch": B, "context": context, "new_tokens": new,
            "note": "wall clock around gmoe_model_forward_token (each a synchronised step with its logits copied "
                    "to the host) and gmoe_model_prefill; glm.c's CPU forward at the same position: "
                    "python3 bench.py --e2e --e2e-cpu"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=N_MOE_LAYERS)
    ap.add_argument("--profile-steps", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extras", action="store_true",
                    help="only the headline decode stack (no single-layer, prefill or drop-in hook timings)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device-to-device 5 times (calibrates the PMC byte counters)")
    ap.add_argument("--prefill", type=int, default=0, metavar="T",
                    help="instead of decode, time one MoE layer over T tokens (the grouped expert GEMM path)")
    ap.add_argument("--zipf", action="store_true", help="with --prefill: Zipf(1.2)-skewed router bias")
    ap.add_argument("--prefill-layers", type=int, default=8, help="seeded layers the prefill timings rotate through")
    ap.add_argument("--group-size", type=int, default=32, choices=(16, 32),
                    help="16: the exporter's form (fp32 scales); with --prefill that prefill workload, alone the "
                         "46-layer decode step and a T=512 prefill layer")
    ap.add_argument("--e2e", action="store_true",
                    help="only the whole-model decode (a --context-token prompt by batched prefill, then --new tokens)")
    ap.add_argument("--context", type=int, default=4096)
    ap.add_argument("--prefill-batch", type=int, default=PREFILL_BATCH,
                    help="with --e2e: prompt tokens per batched prefill step (the MoE context's max_tokens)")
    ap.add_argument("--new", type=int, default=128)
    ap.add_argument("--e2e-cpu", action="store_true",
                    help="with --e2e: also time glm.c's CPU forward at the same position (writes a ~33 GB checkpoint "
                         "to a RAM-backed temporary file for the run)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (expert-parallel sharding is "
              "design-only); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import gmoe

    if args.copy_probe:
        n = args.copy_probe << 20
        src, dst = gmoe.DeviceArray(n), gmoe.DeviceArray(n)
        gmoe.hip_check(gmoe.hip().hipMemset(src.ptr, 1, n), "hipMemset")
        for _ in range(5):
            gmoe.hip_check(gmoe.hip().hipMemcpy(dst.ptr, src.ptr, n, gmoe.HIP_D2D), "hipMemcpy D2D")
        gmoe.hip_check(gmoe.hip().hipDeviceSynchronize(), "sync")
        print(json.dumps({"copy_probe_bytes": n, "copies": 5}), flush=True)
        return

    if args.prefill:
        return prefill_only(args, gmoe, np)
    if args.e2e:
        return e2e_only(args, gmoe, np)
    if args.group_size == 16:
        return gs16_only(args, gmoe, np)

    shape = gmoe.GLM47_FLASH
    L = args.layers
    if gmoe.device_count() < 1:
        raise SystemExit("no HIP device visible")
    extras = not args.no_extras
    max_tokens = PREFILL_BATCH if extras else 1

    t0 = time.perf_counter()
    ctx = gmoe.Context(shape, n_layers=L + 1, max_tokens=max_tokens, device=0)
    keep = not args.no_cpu or extras
    host_layers = []
    for layer in range(1, L + 1):
        hl = gmoe.HostLayer(shape, seed=0, layer=layer)
        ctx.upload(layer, hl)
        if keep:
            host_layers.append(hl)
        else:
            del hl
    log(f"generated and uploaded {L} layers in {time.perf_counter() - t0:.1f}s")

    x0 = gmoe.activations(0, 0, 1, shape.D)
    d_in = gmoe.DeviceArray.from_numpy(x0)
    d_out = gmoe.DeviceArray(x0.nbytes)
    stream = gmoe.Stream()

    def step():
        ctx.forward_layers(1, L, 1, d_in.ptr, d_out.ptr, stream=stream.h)

    for _ in range(args.warmup):
        step()
    stream.sync()
    gmoe.hip_check(gmoe.hip().hipDeviceSynchronize(), "sync")
    t_begin = time.perf_counter()
    for _ in range(args.steps):
        step()
    stream.sync()
    gmoe.hip_check(gmoe.hip().hipDeviceSynchronize(), "sync")
    elapsed = time.perf_counter() - t_begin
    ms_per_step = elapsed * 1e3 / args.steps
    tokens_per_s = args.steps / elapsed
    stats = ctx.stats()  # also reports a timed-out launch of the timed steps as an error
    bytes_per_token = 0
    for layer in range(1, L + 1):
        idx, _ = ctx.read_topk(layer, 1)
        bytes_per_token += (int(np.sum(idx >= 0)) + 1) * shape.expert_bytes()
    layer_us = ms_per_step * 1e3 / L
    stack_gbs = bytes_per_token / (ms_per_step * 1e-3) / 1e9
    log(f"{tokens_per_s:.1f} tok/s, {layer_us:.2f} us/layer, {stack_gbs:.0f} GB/s on expert bytes")

    # per-token latencies (glm.c's bench-mode p50/p95): each step of a separate pass of
    # args.steps steps between HIP events on the stream, with no host synchronisation inside
    ev = [gmoe.Event() for _ in range(args.steps + 1)]
    ev[0].record(stream)
    for i in range(args.steps):
        step()
        ev[i + 1].record(stream)
    stream.sync()
    per_token = latency_stats([ev[i].elapsed_ms(ev[i + 1]) for i in range(args.steps)])
    per_token["note"] = "HIP events between consecutive steps of a second pass of the same steps"

    # per-kernel HIP-event timing over a separate pass of the same steps
    ctx.profile(True)
    for _ in range(args.profile_steps):
        step()
    stream.sync()
    prof = ctx.profile_read()
    ctx.profile(False)
    if not prof:
        raise SystemExit("--profile-steps must be at least 1: the roofline needs the kernel's launch time")
    K1 = shape.K + 1
    mat = shape.F * shape.D * 34 // 32
    kernel_bytes = {"gate_up": K1 * 2 * mat, "down": K1 * mat, "k_moe_stack": bytes_per_token,
                    "k_moe_relay": bytes_per_token}
    dom = max(prof, key=lambda k: prof[k][1])
    kernels = {k: {"launches": n, "avg_us": ms * 1e3 / n} for k, (n, ms) in prof.items()}
    for k in kernels:
        if k in kernel_bytes:
            kernels[k]["bytes_per_launch"] = kernel_bytes[k]
            kernels[k]["gbs"] = kernel_bytes[k] / (kernels[k]["avg_us"] * 1e-6) / 1e9
    dom_bytes = kernel_bytes.get(dom, 0)
    dom_us = kernels[dom]["avg_us"]
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9 if dom_bytes else 0.0
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(dom),
                "bytes_per_launch": dom_bytes, "avg_launch_us": round(dom_us, 3)}

    extra = {}
    if extras:
        # config 1: one MoE layer per launch, rotating over the resident layers so that no
        # layer's experts are still cached from the launch before
        it = [0]

        def one_layer():
            lay = 1 + it[0] % L
            ctx.forward_layers(lay, 1, 1, d_in.ptr, d_out.ptr, stream=stream.h)
            it[0] += 1

        for _ in range(L):
            one_layer()
        stream.sync()
        us = hip_events_us(gmoe, stream, one_layer, 4 * L)
        lb = (shape.K + 1) * shape.expert_bytes()
        extra["single_layer"] = {
            "workload": "one GLM-4.7-Flash MoE layer per launch, T=1, rotating over the 46 resident layers",
            "layer_us": round(us, 3), "expert_bytes": lb, "hbm_gbps": round(lb / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(lb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "launches": 4 * L}
        log(f"single layer: {us:.2f} us")
        # configs 3 and 4: prefill batches on the grouped expert GEMMs
        NL = min(args.prefill_layers, L)
        x512 = gmoe.activations(0, 1, 512, shape.D)
        extra["prefill_t512"] = time_prefill(gmoe, np, ctx, shape, list(range(1, NL + 1)), 512, x512,
                                             max(2, args.warmup), max(10, args.steps), 10)
        extra["prefill_t512"]["workload"] = f"one GLM-4.7-Flash MoE layer, T=512, N(0, 0.01) bias, {NL} layers rotated"
        log(f"prefill T=512: {extra['prefill_t512']['layer_us']} us/layer")
        zctx = gmoe.Context(shape, n_layers=NL + 1, max_tokens=128, device=0)
        zipf_l1 = None
        for layer in range(1, NL + 1):
            hl = gmoe.HostLayer(shape, seed=0, layer=layer, bias_mode=gmoe.SYNTH_BIAS_ZIPF)
            zctx.upload(layer, hl)
            if layer == 1:
                zipf_l1 = hl
        x128 = gmoe.activations(0, 1, 128, shape.D)
        extra["prefill_t128_zipf"] = time_prefill(gmoe, np, zctx, shape, list(range(1, NL + 1)), 128, x128,
                                                  max(2, args.warmup), max(10, args.steps), 10)
        extra["prefill_t128_zipf"]["workload"] = f"one GLM-4.7-Flash MoE layer, T=128, Zipf(1.2) bias, {NL} layers rotated"
        zstats = zctx.stats()
        zctx.close()
        log(f"prefill T=128 Zipf: {extra['prefill_t128_zipf']['layer_us']} us/layer")
        if not args.no_cpu:
            extra["prefill_t512"]["cpu_baseline"] = cpu_prefill_baseline(shape, host_layers[0], x512)
            extra["prefill_t128_zipf"]["cpu_baseline"] = cpu_prefill_baseline(shape, zipf_l1, x128)
        extra["prefill_t128_zipf"]["routing_stats"] = zstats
        del zipf_l1
        # the glm.c drop-in hook on host memory (uploads its own copy of the layers)
        extra["backend_hook"] = backend_hook_us(gmoe, np, shape, host_layers, x0)
        log(f"backend hook: {extra['backend_hook']['layer_us']} us/layer")
        extra["gs16"] = gs16_form(gmoe, np, args, L)
        log(f"gs16: {extra['gs16']['decode_tokens_s']} tok/s decode, "
            f"{extra['gs16']['prefill_t512']['layer_us']} us/layer prefill T=512")
        if L == N_MOE_LAYERS:
            extra["e2e_decode"] = e2e_decode(gmoe, np, ctx)
            log(f"e2e: {extra['e2e_decode']['decode_tokens_s']} tok/s decode, "
                f"{extra['e2e_decode']['prefill_tokens_s']} tok/s prefill")
            if not args.no_cpu:
                log("e2e: timing glm.c's CPU forward at position 4096")
                extra["e2e_decode"]["cpu_baseline"] = e2e_cpu_baseline(gmoe, 4096)

    cpu = None
    if not args.no_cpu:
        log(f"timing the CPU reference path for ~{args.cpu_seconds:.0f}s")
        cpu = cpu_baseline(shape, host_layers, x0, args.cpu_seconds)

    out = {
        "metric": METRIC,
        "value": round(tokens_per_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint8->int32 + fp32",
        "data": "synthetic (seeded random-init Q8_0 weights, N(0,1) input)",
        "config": {"workload": "GLM-4.7-Flash MoE stack decode: 46 MoE layers, T=1", "layers": L, "tokens_per_step": 1,
                   "dim": shape.D, "moe_ffn_dim": shape.F, "experts": shape.E, "top_k": shape.K, "shared_experts": 1,
                   "quant": "Q8_0 (32 x int8 + fp16 scale)", "seed": 0},
        "layer_us": round(layer_us, 3),
        "per_token": per_token,
        "expert_bytes_per_token": bytes_per_token,
        "hbm_gbps_expert_bytes": round(stack_gbs, 1),
        "hbm_frac_expert_bytes": round(stack_gbs / HBM_PEAK_GBS, 4),
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "routing_stats": stats,
        **extra,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


E2E_CPU_SCRIPT = r"""
import ctypes as C, json, sys
lib = C.CDLL(sys.argv[1])
lib.ref_forward_timed.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double)]
lib.ref_forward_timed.restype = C.c_int
pos, cap, n, threads = (int(v) for v in sys.argv[3:7])
ms = (C.c_double * n)()
rc = lib.ref_forward_timed(sys.argv[2].encode(), 5, pos, cap, n, threads, ms)
print(json.dumps({"rc": rc, "token_ms": list(ms)}))
"""


def e2e_cpu_baseline(gmoe, context, tokens=2):
    """glm.c's own CPU forward (oracle/_ref: infer.c's glm_cpu_forward_token, its Makefile's
    flags, OpenMP bound to cores) on a synthetic v4 checkpoint of the same GLM-4.7-Flash
    shape, `tokens` tokens at position `context` of a zeroed cache (the attention reads
    every earlier position either way), in a child process since glm.c's loader exits on
    a file it rejects. The checkpoint (~33 GB) lives in a RAM-backed temporary file for
    the run only."""
    import tempfile
    import glm_model
    import oracle
    if not oracle.available("reference"):
        return None
    m = gmoe.GLM47_FLASH_MODEL
    sp = glm_model.CkptSpec(dim=m["dim"], hidden_dim=m["hidden_dim"], n_layers=m["n_layers"], n_heads=m["n_heads"],
                            n_kv_heads=m["n_heads"], vocab_size=m["vocab_size"], seq_len=context + tokens + 8,
                            rope_dim=m["rope_dim"], q_lora_rank=m["q_lora_rank"], kv_lora_rank=m["kv_lora_rank"],
                            n_routed_experts=64, n_experts_used=4, bos_id=1, eos_id=2, qk_nope_dim=m["qk_nope_dim"],
                            v_head_dim=m["v_head_dim"], moe_ffn_dim=1536, group_size=m["group_size"], seed=0,
                            norm_mode=gmoe.SYNTH_NORM_RANDOM, bias_mode=gmoe.SYNTH_BIAS_NORMAL,
                            scale_mode=gmoe.SYNTH_SCALES_FP16)
    tmp_dir = "/dev/shm" if os.path.isdir("/dev/shm") else None
    fd, path = tempfile.mkstemp(prefix="glm_e2e_", suffix=".bin", dir=tmp_dir)
    os.close(fd)
    try:
        t0 = time.perf_counter()
        glm_model.write_synth_checkpoint(path, sp)
        log(f"e2e CPU: wrote a {os.path.getsize(path) / 1e9:.1f} GB checkpoint in {time.perf_counter() - t0:.1f}s")
        threads = omp_threads()
        r = subprocess.run([sys.executable, "-c", E2E_CPU_SCRIPT, oracle.PATHS["reference"], path, str(context),
                            str(context + tokens + 1), str(tokens), str(threads)], capture_output=True, text=True,
                           timeout=900)
        if r.returncode != 0:
            raise SystemExit(f"glm.c's CPU forward failed: {r.stdout[-2000:]} {r.stderr[-2000:]}")
        res = json.loads(r.stdout.strip().splitlines()[-1])
        if res["rc"] != 0:
            raise SystemExit("glm.c's CPU forward returned an error")
    finally:
        os.unlink(path)
    ms = median(res["token_ms"])
    return {"value": round(1e3 / ms, 4), "unit": "tokens/s", "cores": threads, "kind": "reference",
            "sample": f"{tokens} decode tokens at position {context} of glm.c's CPU forward (infer.c built with its "
                      f"Makefile flags, OpenMP threads bound to cores) on a synthetic checkpoint of the same shape; "
                      f"median per-token time",
            "ms_per_token": round(ms, 1), "token_ms": [round(v, 1) for v in res["token_ms"]]}


def e2e_only(args, gmoe, np):
    """--e2e: the whole-model decode alone, on 46 freshly uploaded MoE layers."""
    shape = gmoe.GLM47_FLASH
    t0 = time.perf_counter()
    ctx = gmoe.Context(shape, n_layers=N_MOE_LAYERS + 1, max_tokens=args.prefill_batch, device=0)
    for layer in range(1, N_MOE_LAYERS + 1):
        ctx.upload(layer, gmoe.HostLayer(shape, seed=0, layer=layer))
    log(f"generated and uploaded {N_MOE_LAYERS} layers in {time.perf_counter() - t0:.1f}s")
    res = e2e_decode(gmoe, np, ctx, context=args.context, new=args.new)
    ctx.close()
    cpu = None
    if args.e2e_cpu:
        log(f"timing glm.c's CPU forward at position {args.context}")
        cpu = e2e_cpu_baseline(gmoe, args.context)
    out = {
        "metric": "GLM-4.7-Flash-shaped model decode tokens/s (47 layers, Q8_0, whole forward on the GPU)",
        "value": res["decode_tokens_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.new,
        "warmup": 2,
        "ms_per_step": res["decode_ms_per_token"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights; fp32 attention and activations",
        "data": "synthetic (seeded random-init Q8_0 weights, random prompt tokens)",
        "config": {"workload": res["workload"], "context": args.context, "new_tokens": args.new},
        **{k: v for k, v in res.items() if k not in ("workload", "decode_tokens_s", "decode_ms_per_token")},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def prefill_only(args, gmoe, np):
    """--prefill T: one MoE layer over T tokens (T=512 with N(0, 0.01) router bias, or
    T=128 with the Zipf(1.2) bias), the workload of the prefill profiles."""
    shape = gmoe.Shape(group_size=args.group_size)
    T, NL = args.prefill, args.prefill_layers
    bias = gmoe.SYNTH_BIAS_ZIPF if args.zipf else gmoe.SYNTH_BIAS_NORMAL
    scales = gmoe.SYNTH_SCALES_FP16 if args.group_size == 32 else gmoe.SYNTH_SCALES_FP32
    t0 = time.perf_counter()
    ctx = gmoe.Context(shape, n_layers=NL + 1, max_tokens=T, device=0)
    first = None
    for layer in range(1, NL + 1):
        hl = gmoe.HostLayer(shape, seed=0, layer=layer, bias_mode=bias, scale_mode=scales)
        ctx.upload(layer, hl)
        if layer == 1:
            first = hl
    log(f"generated and uploaded {NL} layers in {time.perf_counter() - t0:.1f}s")
    x0 = gmoe.activations(0, 1, T, shape.D)
    res = time_prefill(gmoe, np, ctx, shape, list(range(1, NL + 1)), T, x0, args.warmup, args.steps,
                       args.profile_steps)
    cpu = None if args.no_cpu else cpu_prefill_baseline(shape, first, x0)
    name = f"T={T}" + (" Zipf(1.2) routing" if args.zipf else "") + ("" if args.group_size == 32 else
                                                                    f", group size {args.group_size} fp32 scales")
    out = {
        "metric": f"MoE-layer prefill tokens/s ({name}, GLM-4.7-Flash shape, Q8_0, grouped expert GEMM)",
        "value": res["tokens_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["layer_us"] * 1e-3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 x (int8 as fp16) MFMA, fp32 accumulate (activations as fp16 hi+lo)",
        "data": "synthetic (seeded random-init Q8_0 weights, N(0,1) input)",
        "config": {"workload": f"one GLM-4.7-Flash MoE layer, prefill {name}", "tokens": T, "layers_rotated": NL,
                   "dim": shape.D, "moe_ffn_dim": shape.F, "experts": shape.E, "top_k": shape.K, "shared_experts": 1},
        **{k: v for k, v in res.items() if k != "tokens_s"},
        "cpu_baseline": cpu,
        "routing_stats": ctx.stats(),
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
