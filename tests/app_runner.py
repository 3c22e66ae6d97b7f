"""glm.c's own command-line app (infer.c:1985-2262) on synthetic checkpoints, in the two
builds oracle/build_app.py makes from the reference sources: `glm-cpu` (the reference app as
its Makefile builds it) and `glm-hip` (the same app with the drop-in patch, linked against
libglm_hip.so in place of backend.c). Both are run as child processes; their generated text
and bench reports are what the tests compare."""
import json
import os
import subprocess

import glm_model
import gmoe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_OUT = os.path.join(ROOT, "oracle", "_ref")
APPS = {"cpu": os.path.join(REF_OUT, "glm-cpu"), "hip": os.path.join(REF_OUT, "glm-hip")}
REF_DIR = "/root/reference"
PROMPT = "thequickbrownfoxjumpsoverthelazydog"


def available():
    """Whether both binaries exist, building them first where the reference sources are."""
    if not all(os.path.exists(p) for p in APPS.values()) and os.path.isfile(os.path.join(REF_DIR, "infer.c")):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "app", f"REF_DIR={REF_DIR}"], check=True,
                       capture_output=True)
    return all(os.path.exists(p) for p in APPS.values())


def small_spec(seed=5, n_layers=3, seq_len=128):
    return glm_model.CkptSpec(dim=256, hidden_dim=512, n_layers=n_layers, n_heads=4, n_kv_heads=4, vocab_size=300,
                              seq_len=seq_len, rope_dim=16, q_lora_rank=64, kv_lora_rank=64, n_routed_experts=8,
                              n_experts_used=2, bos_id=1, eos_id=2, qk_nope_dim=32, v_head_dim=32, moe_ffn_dim=256,
                              group_size=32, seed=seed, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                              bias_mode=gmoe.SYNTH_BIAS_NORMAL, scale_mode=gmoe.SYNTH_SCALES_FP16)


def write_model(directory, spec):
    path = os.path.join(str(directory), "model.bin")
    glm_model.write_synth_checkpoint(path, spec)
    glm_model.write_tokenizer(path + ".tokenizer", spec.vocab_size, spec.bos_id, spec.eos_id)
    return path


def run(app, model, args, env=None, timeout=300):
    e = dict(os.environ)
    e.setdefault("OMP_NUM_THREADS", "4")
    if env:
        e.update(env)
    return subprocess.run([APPS[app], model] + list(args), capture_output=True, text=True, timeout=timeout, env=e)


def generated(stdout):
    """The app's output without its banner's backend line (infer.c:2087)."""
    return [ln for ln in stdout.splitlines() if not ln.strip().startswith("backend=")]


def bench_report(path):
    with open(path) as f:
        return json.load(f)
