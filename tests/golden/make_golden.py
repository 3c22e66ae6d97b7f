#!/usr/bin/env python3
"""Write the golden fixtures of the MoE path from glm.c's own code.

Every expected output here comes from oracle/_ref/libref_moe.so: glm.c's infer.c
(apply_moe_shared_ffn_layer, infer.c:1087-1216) compiled from the reference
sources by `make -C oracle ref`. glm.c ships no test vectors for this path, so
these fixtures are what pins the CPU restatement (oracle/moe_oracle.c) and, at
full size, the GPU path. Inputs are the seeded synthetic tensors of
glm.c_amd/host/synth.c; each fixture stores the SHA-256 of the weights it used,
so a change in the generator shows up as a fixture mismatch, not as a silent
change of workload.

    python tests/golden/make_golden.py      # needs oracle/_ref/libref_moe.so

Fixtures (numpy .npz, no pickles):
  small.npz             D=256 F=256 E=16 K=4, T=4: every intermediate, plus a
                        variant with exact router ties and a NaN router row,
                        the routed-experts-off variant and a 3-layer stack
  glm_t1.npz            GLM-4.7-Flash layer 1 (D=2048 F=1536 E=64 K=4), T=1:
                        xn, router p[64], top-k, shared and routed outputs, x_out
  dispatch_t128_zipf.npz  T=128 with Zipf-shaped router bias: per-token top-k,
                        per-expert token lists, sampled output rows, checksums
  dispatch_t512.npz     T=512, N(0, 0.01) bias: the same
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for sub in ("glm.c_amd", "oracle", "tests"):
    sys.path.insert(0, os.path.join(ROOT, sub))

import gmoe  # noqa: E402
import oracle  # noqa: E402
from golden_data import SMALL, with_ties_and_nan  # noqa: E402

SAMPLE_ROWS = {128: [0, 1, 63, 64, 126, 127], 512: [0, 1, 255, 256, 510, 511]}


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def weight_digests(hl, experts):
    """SHA-256 of the router, the shared expert and the listed routed experts."""
    d = {"gate_inp": sha(hl.gate_inp), "exp_probs_b": sha(hl.exp_probs_b), "ffn_norm": sha(hl.ffn_norm)}
    for n in ("gate_sh_q", "gate_sh_s", "up_sh_q", "up_sh_s", "down_sh_q", "down_sh_s"):
        d[n] = sha(getattr(hl, n))
    for e in experts:
        for n in ("gate_q", "gate_s", "up_q", "up_s", "down_q", "down_s"):
            d[f"{n}[{e}]"] = sha(getattr(hl, n)[e])
    return d


def digest_arrays(d):
    keys = sorted(d)
    return np.array(keys), np.array([d[k] for k in keys])


def small(ref):
    out = {}
    hl = gmoe.HostLayer(SMALL, seed=7, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    x = gmoe.activations(7, 0, 4, SMALL.D)
    out["x"] = x
    for k, v in ref.layer(SMALL, hl, x).items():
        out[k] = v
    out["off_x_out"] = ref.layer(SMALL, hl, x, disable_routed=True)["x_out"]
    tk = with_ties_and_nan(gmoe.HostLayer(SMALL, seed=7, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM))
    for k, v in ref.layer(SMALL, tk, x).items():
        out["tie_" + k] = v
    layers = [gmoe.HostLayer(SMALL, seed=11, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM) for l in (1, 2, 3)]
    xs, topk = ref.stack(SMALL, layers, x)
    out["stack_x_out"], out["stack_topk_idx"] = xs, topk
    out["digest_keys"], out["digest_values"] = digest_arrays(weight_digests(hl, range(SMALL.E)))
    return out


def glm_t1(ref):
    s = gmoe.GLM47_FLASH
    hl = gmoe.HostLayer(s, seed=0, layer=1)
    x = gmoe.activations(0, 0, 1, s.D)
    res = ref.layer(s, hl, x)
    out = {"x": x, **res}
    sel = sorted(set(res["topk_idx"].ravel().tolist()) | {0, s.E - 1})
    out["digest_keys"], out["digest_values"] = digest_arrays(weight_digests(hl, sel))
    return out


def dispatch_case(ref, T, stream, bias_mode):
    s = gmoe.GLM47_FLASH
    hl = gmoe.HostLayer(s, seed=0, layer=1, bias_mode=bias_mode)
    x = gmoe.activations(0, stream, T, s.D)
    res = ref.layer(s, hl, x)
    offsets, tokens, slots = oracle.dispatch(res["topk_idx"], s.E)
    rows = SAMPLE_ROWS[T]
    x_out = res["x_out"].astype(np.float64)
    counts = np.diff(offsets)
    out = {"x_rows": x[rows], "rows": np.array(rows, np.int32), "topk_idx": res["topk_idx"], "topk_w": res["topk_w"],
           "offsets": offsets, "tokens": tokens, "slots": slots, "x_out_rows": res["x_out"][rows],
           "x_out_sum": np.array(x_out.sum()), "x_out_sumsq": np.array((x_out * x_out).sum()),
           "x_out_row_sums": res["x_out"].astype(np.float64).sum(axis=1),
           "top4_share": np.array(np.sort(counts)[::-1][:4].sum() / max(1, counts.sum())),
           "n_touched": np.array(int((counts > 0).sum()))}
    out["digest_keys"], out["digest_values"] = digest_arrays(weight_digests(hl, [0, s.E - 1]))
    return out


def main():
    if not oracle.available("reference"):
        raise SystemExit("oracle/_ref/libref_moe.so is missing: run `make -C oracle ref` first")
    ref = oracle.Oracle("reference")
    jobs = [("small.npz", lambda: small(ref)), ("glm_t1.npz", lambda: glm_t1(ref)),
            ("dispatch_t128_zipf.npz", lambda: dispatch_case(ref, 128, 1, gmoe.SYNTH_BIAS_ZIPF)),
            ("dispatch_t512.npz", lambda: dispatch_case(ref, 512, 2, gmoe.SYNTH_BIAS_NORMAL))]
    only = set(sys.argv[1:])
    for name, fn in jobs:
        if only and name not in only:
            continue
        data = fn()
        np.savez_compressed(os.path.join(HERE, name), **data)
        print(f"wrote {name}: " + ", ".join(f"{k}{list(np.shape(v))}" for k, v in data.items()), flush=True)


if __name__ == "__main__":
    main()
