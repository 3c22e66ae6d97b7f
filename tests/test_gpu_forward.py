"""glm.c's token forward through the HIP backend (glm_hip_forward_token, what
glm_backend_forward_token runs for BACKEND_HIP) against glm.c's own forward
(infer.c:1767-1901, compiled into oracle/_ref) on synthetic v4 checkpoints, in both forms
the backend takes:

* "gpu": the whole forward on the GPU model (gmoe_model.h): embedding, MLA attention over
  the device-resident latent cache, dense layer 0, the MoE layers, LM head;
* "host_attn" (GLM_HIP_HOST_ATTN=1): glm.c's host steps around the GPU MoE layers.

Teacher-forced: the same tokens at the same positions on both sides, with glm.c's dual
checkpoints (infer.c:1940-1983) per position. Every checkpoint and the logits are held to
the FFN bar, max-abs 1e-2 and rel-L2 1e-3, and each position's argmax equals glm.c's. In
the host form layer 0 (attention and dense FFN) never sees a GPU result, so its
checkpoints equal glm.c's bit for bit at every position.

Greedy: the decoder picks each next token itself (argmax, with infer.c:2213-2219's
bos/eos skips), and glm.c, fed the same sequence, picks the same token at every step.
A 150-position run takes the GPU attention over several 32-position chunks."""
import numpy as np
import pytest

import glm_model
import gmoe
import ref_decode
from conftest import assert_close

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not ref_decode.available(), reason="oracle/_ref not built (needs the reference sources)")]


def small(gs, scale_mode, n_layers=4, seed=21, seq_len=64):
    return glm_model.CkptSpec(dim=256, hidden_dim=512, n_layers=n_layers, n_heads=4, n_kv_heads=4, vocab_size=300,
                              seq_len=seq_len, rope_dim=16, q_lora_rank=64, kv_lora_rank=64, n_routed_experts=8,
                              n_experts_used=2, bos_id=1, eos_id=2, qk_nope_dim=32, v_head_dim=32, moe_ffn_dim=256,
                              group_size=gs, seed=seed, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                              bias_mode=gmoe.SYNTH_BIAS_NORMAL, scale_mode=scale_mode)


def glm_dims(seed=22):
    """GLM-4.7-Flash's MoE dimensions (D 2048, F 1536, 64 experts, top-4, group size 32)
    and attention ranks (kv_lora 512, rope 64, nope 192, v_head 256), with a small
    vocabulary, four heads and two MoE layers."""
    return glm_model.CkptSpec(dim=2048, hidden_dim=1024, n_layers=3, n_heads=4, n_kv_heads=4, vocab_size=1000,
                              seq_len=64, rope_dim=64, q_lora_rank=256, kv_lora_rank=512, n_routed_experts=64,
                              n_experts_used=4, bos_id=1, eos_id=2, qk_nope_dim=192, v_head_dim=256, moe_ffn_dim=1536,
                              group_size=32, seed=seed, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                              bias_mode=gmoe.SYNTH_BIAS_NORMAL, scale_mode=gmoe.SYNTH_SCALES_FP16)


def glm_heads(seed=25):
    """glm_dims with GLM-4.7-Flash's 20 heads: the attention spreads them over two blocks of
    10 per cache chunk."""
    sp = glm_dims(seed)
    sp.n_heads = sp.n_kv_heads = 20
    return sp


def odd_heads(seed=26):
    """Five heads, so that the attention's last pair of heads has one member."""
    sp = small(32, gmoe.SYNTH_SCALES_FP16, n_layers=3, seed=seed)
    sp.n_heads = sp.n_kv_heads = 5
    return sp


CASES = {"gs16": lambda: small(16, gmoe.SYNTH_SCALES_FP32), "gs32_tiled": lambda: small(32, gmoe.SYNTH_SCALES_FP16),
         "glm_dims": glm_dims, "glm_heads": glm_heads, "odd_heads": odd_heads}
TOKENS = [1, 5, 17, 299, 42, 0, 17, 123, 7, 250]
MODES = ["gpu", "host_attn"]


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.fixture(params=MODES)
def mode(request, monkeypatch):
    if request.param == "host_attn":
        monkeypatch.setenv("GLM_HIP_HOST_ATTN", "1")
    else:
        monkeypatch.delenv("GLM_HIP_HOST_ATTN", raising=False)
    return request.param


def open_decoder(tmp_path, sp, cap, mode):
    path = tmp_path / "model.bin"
    glm_model.write_synth_checkpoint(path, sp)
    ck = glm_model.Checkpoint(path)
    dec = glm_model.Decoder(ck, cap)
    assert dec.backend == glm_model.BACKEND_HIP
    assert dec.on_gpu() == (mode == "gpu"), "the forward runs where the mode says"
    return path, ck, dec


def check_position(dec, ref, pos, logits, attn, layer, mode, what):
    if mode == "host_attn":
        assert np.array_equal(bits(attn[0]), bits(ref["attn"][pos][0])), f"{what}: layer 0 attention"
        assert np.array_equal(bits(layer[0]), bits(ref["layer"][pos][0])), f"{what}: layer 0 FFN"
    for l in range(dec.L):
        assert_close(attn[l], ref["attn"][pos][l], f"{what} layer {l} attention")
        assert_close(layer[l], ref["layer"][pos][l], f"{what} layer {l} FFN")
    assert_close(logits, ref["logits"][pos], f"{what} logits")
    assert int(np.argmax(logits)) == int(np.argmax(ref["logits"][pos])), f"{what}: argmax"


@pytest.mark.parametrize("case", list(CASES))
def test_teacher_forced_positions_match_glm(tmp_path, case, mode):
    sp = CASES[case]()
    tokens = [t % sp.vocab_size for t in TOKENS]
    cap = len(tokens) + 2
    path, ck, dec = open_decoder(tmp_path, sp, cap, mode)
    try:
        ref = ref_decode.reference_decode(path, tokens, cap, dec.L, dec.D, dec.V, tmp_path / "ref")
        for pos, tok in enumerate(tokens):
            print(f"[case] forward {case} {mode} pos {pos} token {tok}", flush=True)
            logits, attn, layer = dec.step(tok, pos, checkpoints=True)
            check_position(dec, ref, pos, logits, attn, layer, mode, f"pos {pos}")
    finally:
        dec.free()
        ck.close()


def test_long_context_over_several_attention_chunks(tmp_path, mode):
    sp = small(32, gmoe.SYNTH_SCALES_FP16, n_layers=3, seed=23, seq_len=256)
    rng = np.random.default_rng(23)
    tokens = [1] + [int(t) for t in rng.integers(3, sp.vocab_size, 149)]
    cap = len(tokens) + 1
    path, ck, dec = open_decoder(tmp_path, sp, cap, mode)
    try:
        ref = ref_decode.reference_decode(path, tokens, cap, dec.L, dec.D, dec.V, tmp_path / "ref")
        print(f"[case] long context {mode}: {len(tokens)} positions", flush=True)
        for pos, tok in enumerate(tokens):
            full = pos in (0, 63, 64, 65, 127, 128, len(tokens) - 1)
            if full:
                logits, attn, layer = dec.step(tok, pos, checkpoints=True)
                check_position(dec, ref, pos, logits, attn, layer, mode, f"pos {pos}")
            else:
                logits = dec.step(tok, pos)
                assert_close(logits, ref["logits"][pos], f"pos {pos} logits")
    finally:
        dec.free()
        ck.close()


def next_token(logits, sp):
    """infer.c:2212-2219 at temperature 0 (bench mode: eos is skipped, not a stop)."""
    t = int(np.argmax(logits))
    if t == sp.bos_id:
        t = (t + 1) % sp.vocab_size
    if t == sp.eos_id:
        t = (t + 1) % sp.vocab_size
    return t


@pytest.mark.parametrize("case", ["gs32_tiled", "glm_dims"])
def test_greedy_decode_picks_glms_tokens(tmp_path, case, mode):
    sp = CASES[case]()
    prompt, n_new = [1, 5, 17], 8
    cap = len(prompt) + n_new + 1
    path, ck, dec = open_decoder(tmp_path, sp, cap, mode)
    try:
        seq, picked = list(prompt), []
        for pos in range(len(prompt) + n_new - 1):
            logits = dec.step(seq[pos], pos)
            if pos + 1 >= len(prompt):
                picked.append(next_token(logits, sp))
                seq.append(picked[-1])
        print(f"[case] greedy {case} {mode}: {seq}", flush=True)
        ref = ref_decode.reference_decode(path, seq, cap, dec.L, dec.D, dec.V, tmp_path / "ref")
        for i, t in enumerate(picked):
            pos = len(prompt) - 1 + i
            assert next_token(ref["logits"][pos], sp) == t, f"step {i} (pos {pos})"
    finally:
        dec.free()
        ck.close()


def test_checkpoints_of_a_state_whose_history_the_model_does_not_hold(tmp_path, monkeypatch):
    """The GPU model's latent cache holds one RunState's history. A second RunState, advanced
    through other tokens, keeps its history in its host cache, so its tokens and its dual
    checkpoints take glm.c's host steps from that cache (layer 0 bit for bit with glm.c),
    and the first state's decode on the GPU model is left as it was."""
    monkeypatch.delenv("GLM_HIP_HOST_ATTN", raising=False)
    import ctypes as C
    sp = small(32, gmoe.SYNTH_SCALES_FP16, n_layers=3, seed=27)
    toks_a, toks_b = [1, 5, 17, 123], [299, 42, 7]
    cap = 8
    path, ck, dec = open_decoder(tmp_path, sp, cap, "gpu")
    lib = dec.lib
    other = glm_model.RunState()
    assert lib.glm_runstate_build(C.byref(other), C.byref(dec.rt), cap) == 0
    try:
        ref_a = ref_decode.reference_decode(path, toks_a, cap, dec.L, dec.D, dec.V, tmp_path / "ref_a")
        ref_b = ref_decode.reference_decode(path, toks_b, cap, dec.L, dec.D, dec.V, tmp_path / "ref_b")
        for pos in range(3):
            dec.step(toks_a[pos], pos)
        for pos in range(2):
            print(f"[case] second state pos {pos}", flush=True)
            assert lib.glm_hip_forward_token(C.byref(dec.rt), C.byref(other), toks_b[pos], pos, 0) == 0
            got = np.ctypeslib.as_array(C.cast(other.logits, C.POINTER(C.c_float)), shape=(dec.V,)).copy()
            assert_close(got, ref_b["logits"][pos], f"second state pos {pos} logits")
        attn = np.zeros((dec.L, dec.D), np.float32)
        layer = np.zeros((dec.L, dec.D), np.float32)
        na, nl = C.c_int(), C.c_int()
        FP = C.POINTER(C.c_float)
        print("[case] dual checkpoints of the second state at pos 2", flush=True)
        assert lib.glm_hip_forward_token_dual_checkpoints(
            C.byref(dec.rt), C.byref(other), toks_b[2], 2, 0, attn.ctypes.data_as(FP), dec.D, dec.L, C.byref(na),
            layer.ctypes.data_as(FP), dec.D, dec.L, C.byref(nl)) == 0
        for l in range(dec.L):
            assert_close(attn[l], ref_b["attn"][2][l], f"second state layer {l} attention")
            assert_close(layer[l], ref_b["layer"][2][l], f"second state layer {l} FFN")
        assert np.array_equal(bits(attn[0]), bits(ref_b["attn"][2][0])), "host steps: layer 0 attention"
        print("[case] first state continues on the GPU model at pos 3", flush=True)
        logits = dec.step(toks_a[3], 3)
        assert_close(logits, ref_a["logits"][3], "first state pos 3 logits")
    finally:
        lib.glm_runstate_free(C.byref(other))
        dec.free()
        ck.close()
