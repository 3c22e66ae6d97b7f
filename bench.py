#!/usr/bin/env python3
"""MoE-stack decode benchmark on one MI355X.

Workload: the MoE half of one GLM-4.7-Flash decode step -- 46 MoE layers in
sequence (hidden 2048, 64 routed experts + 1 shared, moe_intermediate 1536,
top-4, Q8_0 experts), T=1, per-layer seeded synthetic weights resident in HBM
(~30 GB), RMSNorm inside every layer (infer.c:1098). A step is one token through
all 46 layers via gmoe_forward_layers; every step starts from the same input.

Prints one JSON line: tokens/s (value), the per-layer time and the HBM rate on
the selected experts' Q8_0 bytes, the roofline of the dominant kernel (its
HIP-event launch time against MI355X's 8 TB/s) and the reference CPU path timed
on this host (glm.c's own infer.c built from source, OpenMP, same weights).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "glm.c_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
N_MOE_LAYERS = 46
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


def traffic_from_profiles(kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summary, or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return t[kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline(shape, host_layers, x0, seconds):
    """glm.c's CPU MoE path on the same layers: tokens through the 46-layer stack until
    `seconds` of wall time have passed (at least 2 tokens)."""
    import numpy as np
    import oracle

    kind = "reference" if oracle.available("reference") else "port"
    orc = oracle.Oracle(kind)
    x = np.array(x0, np.float32)
    orc.stack(shape, host_layers, x)  # warm the page cache and the thread pool
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        orc.stack(shape, host_layers, x)
        times.append(time.perf_counter() - t0)
        if len(times) >= 2 and time.perf_counter() - t_start >= seconds:
            break
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": 1.0 / med,
        "unit": "tokens/s",
        "cores": omp_threads(),
        "kind": kind,
        "sample": f"{len(times)} decode tokens through the same {len(host_layers)}-layer stack, median of per-token "
                  f"wall times (monotonic clock), OpenMP threads = OMP_NUM_THREADS",
        "ms_per_token": med * 1e3,
        "layer_us": med * 1e6 / len(host_layers),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=N_MOE_LAYERS)
    ap.add_argument("--profile-steps", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device-to-device 5 times (calibrates the PMC byte counters)")
    ap.add_argument("--prefill", type=int, default=0, metavar="T",
                    help="instead of decode, time one MoE layer over T tokens (the grouped expert GEMM path)")
    ap.add_argument("--zipf", action="store_true", help="with --prefill: Zipf(1.2)-skewed router bias")
    ap.add_argument("--prefill-layers", type=int, default=8, help="with --prefill: seeded layers rotated through")
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
        return prefill(args, gmoe, np)

    shape = gmoe.GLM47_FLASH
    L = args.layers
    n_dev = gmoe.device_count()
    if n_dev < 1:
        raise SystemExit("no HIP device visible")

    t0 = time.perf_counter()
    ctx = gmoe.Context(shape, n_layers=L + 1, max_tokens=1, device=0)
    keep = not args.no_cpu
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
    per_layer_bytes = ctx.expert_bytes_last()  # T=1: (K valid + shared) experts of the last layer
    bytes_per_token = 0
    for layer in range(1, L + 1):
        idx, _ = ctx.read_topk(layer, 1)
        bytes_per_token += (int(np.sum(idx >= 0)) + 1) * shape.expert_bytes()
    layer_us = ms_per_step * 1e3 / L
    stack_gbs = bytes_per_token / (ms_per_step * 1e-3) / 1e9
    log(f"{tokens_per_s:.1f} tok/s, {layer_us:.2f} us/layer, {stack_gbs:.0f} GB/s on expert bytes")

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
    kernel_bytes = {"gate_up": K1 * 2 * mat, "down": K1 * mat, "k_moe_stack": bytes_per_token}
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
    stats = ctx.stats()

    cpu = None
    if keep:
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
        "expert_bytes_per_token": bytes_per_token,
        "hbm_gbps_expert_bytes": round(stack_gbs, 1),
        "hbm_frac_expert_bytes": round(stack_gbs / HBM_PEAK_GBS, 4),
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "routing_stats": stats,
        "expert_bytes_last_layer": per_layer_bytes,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16


def prefill(args, gmoe, np):
    """One MoE layer over T tokens (T=512 with N(0, 0.01) router bias, or T=128 with the
    Zipf(1.2) bias): router, dispatch, grouped
    gate/up and down GEMMs, combine. Steps rotate over --prefill-layers seeded layers so
    that no layer's 650 MB of touched experts is still cached from the step before."""
    shape = gmoe.GLM47_FLASH
    T, NL = args.prefill, args.prefill_layers
    bias = gmoe.SYNTH_BIAS_ZIPF if args.zipf else gmoe.SYNTH_BIAS_NORMAL
    t0 = time.perf_counter()
    ctx = gmoe.Context(shape, n_layers=NL + 1, max_tokens=T, device=0)
    host_layers = []
    for layer in range(1, NL + 1):
        hl = gmoe.HostLayer(shape, seed=0, layer=layer, bias_mode=bias)
        ctx.upload(layer, hl)
        host_layers.append(hl if layer == 1 else None)
    log(f"generated and uploaded {NL} layers in {time.perf_counter() - t0:.1f}s")
    x0 = gmoe.activations(0, 1, T, shape.D)
    d_in = gmoe.DeviceArray.from_numpy(x0)
    d_out = gmoe.DeviceArray(x0.nbytes)
    stream = gmoe.Stream()
    it = [0]

    def step():
        ctx.forward(1 + it[0] % NL, T, d_in.ptr, d_out.ptr, stream=stream.h)
        it[0] += 1

    for _ in range(args.warmup):
        step()
    stream.sync()
    t_begin = time.perf_counter()
    for _ in range(args.steps):
        step()
    stream.sync()
    elapsed = time.perf_counter() - t_begin
    layer_us = elapsed * 1e6 / args.steps
    # touched experts and routed pairs of every layer (lists are exact, so this is what was read)
    touched, pairs = [], []
    for layer in range(1, NL + 1):
        _, st = gmoe.forward_host(ctx, layer, x0)
        counts = np.diff(st["expert_offsets"])
        touched.append(int(np.sum(counts > 0)) + 1)
        pairs.append(int(counts.sum()) + T)
    bytes_per_layer = float(np.mean(touched)) * shape.expert_bytes()
    macs = float(np.mean(pairs)) * 3 * shape.F * shape.D
    ctx.profile(True)
    for _ in range(args.profile_steps):
        step()
    stream.sync()
    prof = ctx.profile_read()
    ctx.profile(False)
    kernels = {k: {"launches": n, "avg_us": round(ms * 1e3 / n, 3)} for k, (n, ms) in prof.items()}
    # per layer: one gate/up and one down launch
    gemm_us = sum(kernels[k]["avg_us"] for k in ("gate_up", "down") if k in kernels)
    tflops = 2.0 * macs / (gemm_us * 1e-6) / 1e12 if gemm_us else 0.0
    gbs = bytes_per_layer / (layer_us * 1e-6) / 1e9

    cpu = None
    if not args.no_cpu:
        import oracle
        kind = "reference" if oracle.available("reference") else "port"
        orc = oracle.Oracle(kind)
        n = min(T, 32)
        orc.layer(shape, host_layers[0], x0[:2])
        t_c = time.perf_counter()
        orc.layer(shape, host_layers[0], x0[:n])
        dt = time.perf_counter() - t_c
        cpu = {"value": round(n / dt, 2), "unit": "tokens/s", "cores": omp_threads(), "kind": kind,
               "sample": f"{n} of the {T} tokens through layer 1 (glm.c routes prefill tokens one at a time, "
                         f"infer.c:2190-2233), wall clock",
               "layer_us_for_T": round(dt / n * T * 1e6, 1)}
    name = f"T={T}" + (" Zipf(1.2) routing" if args.zipf else "")
    out = {
        "metric": f"MoE-layer prefill tokens/s ({name}, GLM-4.7-Flash shape, Q8_0, grouped expert GEMM)",
        "value": round(T / (layer_us * 1e-6), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(layer_us * 1e-3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 x (int8 as fp16) MFMA, fp32 accumulate (activations as fp16 hi+lo)",
        "data": "synthetic (seeded random-init Q8_0 weights, N(0,1) input)",
        "config": {"workload": f"one GLM-4.7-Flash MoE layer, prefill {name}", "tokens": T, "layers_rotated": NL,
                   "dim": shape.D, "moe_ffn_dim": shape.F, "experts": shape.E, "top_k": shape.K, "shared_experts": 1},
        "layer_us": round(layer_us, 2),
        "touched_experts": round(float(np.mean(touched)), 2),
        "hbm_gbps_touched_bytes": round(gbs, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "mfma": {"algorithmic_tflops": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS, "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                 "note": "algorithmic 2*MACs of the expert products over the two grouped GEMM kernels' time; the "
                         "kernels execute 2x those MACs (hi and lo planes) plus tile padding"},
        "kernels": kernels,
        "cpu_baseline": cpu,
        "routing_stats": ctx.stats(),
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
