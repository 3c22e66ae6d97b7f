"""The drop-in on the GPU, as glm.c drives it.

1. glm.c's backend calls through ctypes: glm_backend_init(BACKEND_HIP) returns the handle,
   glm_backend_forward_token(handle, ...) advances the RunState token by token and fills
   st->logits, glm_backend_free(handle) releases the device (backend.h:7-13,
   backend.c:73-95); the logits are held to glm.c's own forward (oracle/_ref) on the same
   checkpoint.
2. glm.c's own app with the drop-in patch (oracle/_ref/glm-hip, built by
   oracle/build_app.py): `--backend hip` and `GLM_BACKEND=hip` generate, greedily, the text
   that the unpatched reference app generates on the CPU, over a 35-token prompt that the
   patched loop prefills in one batch; glm.c's bench mode reports the HIP run's per-token
   statistics (infer.c:1464-1629)."""
import ctypes as C

import numpy as np
import pytest

import app_runner
import glm_model
import gmoe
import ref_decode
from conftest import assert_close

pytestmark = pytest.mark.gpu
need_ref = pytest.mark.skipif(not ref_decode.available(), reason="oracle/_ref not built (needs the reference sources)")
need_app = pytest.mark.skipif(not app_runner.available(), reason="glm.c's app not built (needs the reference sources)")


@need_ref
def test_backend_forward_token_through_the_returned_handle(tmp_path):
    sp = app_runner.small_spec(seed=9, n_layers=3, seq_len=32)
    path = tmp_path / "model.bin"
    glm_model.write_synth_checkpoint(path, sp)
    ck = glm_model.Checkpoint(path)
    lib = glm_model.forward_lib()
    st = glm_model.RunState()
    tokens = [1, 44, 97, 260, 5, 17]
    cap = len(tokens) + 2
    assert lib.glm_runstate_build(C.byref(st), C.byref(ck.rt), cap) == 0
    handle = None
    try:
        ref = ref_decode.reference_decode(path, tokens, cap, sp.n_layers, sp.dim, sp.vocab_size, tmp_path / "ref")
        print("[case] glm_backend_init(BACKEND_HIP)", flush=True)
        handle = lib.glm_backend_init(glm_model.BACKEND_HIP, C.byref(ck.rt), C.byref(st))
        assert handle == glm_model.BACKEND_HIP
        for pos, tok in enumerate(tokens):
            print(f"[case] glm_backend_forward_token pos {pos}", flush=True)
            assert lib.glm_backend_forward_token(handle, C.byref(ck.rt), C.byref(st), tok, pos, 0) == 0
            logits = np.ctypeslib.as_array(C.cast(st.logits, C.POINTER(C.c_float)), shape=(sp.vocab_size,)).copy()
            assert_close(logits, ref["logits"][pos], f"pos {pos} logits")
            assert int(np.argmax(logits)) == int(np.argmax(ref["logits"][pos])), f"pos {pos} argmax"
        # the CPU handle needs glm.c's own forward, which this process does not link
        assert lib.glm_backend_forward_token(0, C.byref(ck.rt), C.byref(st), 1, 0, 0) == -1
    finally:
        if handle:
            lib.glm_backend_free(handle)
        lib.glm_runstate_free(C.byref(st))
        ck.close()


def glm_shape_spec(seed=12):
    """GLM-4.7-Flash's MoE dimensions and attention ranks, small vocabulary and depth."""
    return glm_model.CkptSpec(dim=2048, hidden_dim=1024, n_layers=3, n_heads=4, n_kv_heads=4, vocab_size=300,
                              seq_len=128, rope_dim=64, q_lora_rank=256, kv_lora_rank=512, n_routed_experts=64,
                              n_experts_used=4, bos_id=1, eos_id=2, qk_nope_dim=192, v_head_dim=256, moe_ffn_dim=1536,
                              group_size=32, seed=seed, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                              bias_mode=gmoe.SYNTH_BIAS_NORMAL, scale_mode=gmoe.SYNTH_SCALES_FP16)


SPECS = {"small": lambda: app_runner.small_spec(seed=5), "glm_shape": glm_shape_spec}


@need_app
@pytest.mark.parametrize("spec", list(SPECS))
def test_app_with_hip_backend_generates_glms_text(tmp_path, spec):
    model = app_runner.write_model(tmp_path, SPECS[spec]())
    args = ["-n", "16", "-i", app_runner.PROMPT, "-t", "0"]
    print(f"[case] glm-cpu {spec}", flush=True)
    ref = app_runner.run("cpu", model, args)
    assert ref.returncode == 0, ref.stderr
    want = app_runner.generated(ref.stdout)
    for extra, env in ((["--backend", "hip"], None), ([], {"GLM_BACKEND": "hip"}),
                       (["--backend", "hip"], {"GLM_HIP_HOST_ATTN": "1"})):
        print(f"[case] glm-hip {spec} {extra} {env}", flush=True)
        got = app_runner.run("hip", model, args + extra, env=env)
        assert got.returncode == 0, got.stderr
        assert "backend=hip" in got.stdout
        assert app_runner.generated(got.stdout) == want, (extra, env)


@need_app
def test_app_bench_mode_reports_the_hip_run(tmp_path):
    model = app_runner.write_model(tmp_path, app_runner.small_spec(seed=6))
    rep = tmp_path / "report.json"
    print("[case] glm-hip --bench-mode full", flush=True)
    r = app_runner.run("hip", model, ["-n", "24", "-i", app_runner.PROMPT, "--bench-mode", "full", "--bench-report",
                                      str(rep), "--backend", "hip"])
    assert r.returncode == 0, r.stderr
    j = app_runner.bench_report(rep)
    assert j["backend"] == "hip"
    assert j["prefill"]["tokens"] == len(app_runner.PROMPT)
    assert j["decode"]["tokens"] >= 20
    for phase in ("prefill", "decode"):
        assert 0 < j[phase]["p50_ms"] <= j[phase]["p95_ms"]


def layer_sums(stderr):
    """glm.c's --debug lines (infer.c:1811-1895, 1207-1210) as (name, value) in print order."""
    out = []
    for ln in stderr.splitlines():
        if ln.startswith("[glm-layer-sum] "):
            name, val = ln[len("[glm-layer-sum] "):].split(" sum=")
            out.append((name, float(val)))
    return out


@need_app
@pytest.mark.parametrize("host_attn", [False, True])
def test_app_debug_mode_prints_glms_layer_sums(tmp_path, host_attn):
    model = app_runner.write_model(tmp_path, app_runner.small_spec(seed=5))
    args = ["-n", "3", "-i", "abcd", "-t", "0", "--debug"]
    ref = app_runner.run("cpu", model, args)
    assert ref.returncode == 0, ref.stderr
    env = {"GLM_HIP_HOST_ATTN": "1"} if host_attn else None
    print(f"[case] glm-hip --debug host_attn={host_attn}", flush=True)
    got = app_runner.run("hip", model, args + ["--backend", "hip"], env=env)
    assert got.returncode == 0, got.stderr
    want, have = layer_sums(ref.stderr), layer_sums(got.stderr)
    assert [n for n, _ in have] == [n for n, _ in want]
    assert len(want) > 25
    for (n, a), (_, b) in zip(have, want):
        assert abs(a - b) <= 0.05 + 1e-3 * abs(b), (n, a, b)
