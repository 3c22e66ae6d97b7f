"""The whole-model decode at the end-to-end workload's own sizes: vocabulary 154,880,
20 heads, q_lora 768, kv_lora 512, rope 64, nope 192, v_head 256, dense layer 0 with
hidden 10,240, GLM-4.7-Flash's MoE layers (D 2048, F 1536, 64 experts, top-4), and a
4,096-token context. Three layers (dense layer 0 and two MoE layers): the MoE depth is
covered by the 46-layer stack tests; here the LM head over all 154,880 rows
(infer.c:1888-1893) and the attention over 4,097 cached positions (infer.c:1017-1058)
are checked at full size.

1. Zeroed cache: glm.c's own forward of a token at position 4096 over runstate_build's
   zeroed cache (infer.c:827-860) against the GPU model from its own zeroed cache: the
   dual checkpoints (x after each layer's attention and FFN) and the logits.
2. After a real 4,096-token batched prefill on the GPU, the next token's dual checkpoints,
   stage by stage against glm.c's own code on the GPU's inputs to that stage: each layer's
   attention (apply_mla_attention_layer) over the latent cache read back from the device,
   each layer's FFN on the GPU's post-attention x, and the final norm and LM head on the
   GPU's last x. Chaining the stages on the device's own values keeps 4,096 positions of
   prefill rounding out of the comparison while every stage is checked at full size.

Every output is held to the FFN bar (max-abs 1e-2, rel-L2 1e-3), and the logits' argmax
must equal glm.c's."""
import ctypes as C
import os

import numpy as np
import pytest

import glm_model
import gmoe
import ref_decode
from conftest import assert_close

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not ref_decode.available(), reason="oracle/_ref not built (needs the reference sources)")]

CTX = 4096
VOCAB = 154880


def config5_spec(n_layers=3, seed=50):
    return glm_model.CkptSpec(dim=2048, hidden_dim=10240, n_layers=n_layers, n_heads=20, n_kv_heads=20,
                              vocab_size=VOCAB, seq_len=CTX + 8, rope_dim=64, q_lora_rank=768, kv_lora_rank=512,
                              n_routed_experts=64, n_experts_used=4, bos_id=1, eos_id=2, qk_nope_dim=192,
                              v_head_dim=256, moe_ffn_dim=1536, group_size=32, seed=seed,
                              norm_mode=gmoe.SYNTH_NORM_RANDOM, bias_mode=gmoe.SYNTH_BIAS_NORMAL,
                              scale_mode=gmoe.SYNTH_SCALES_FP16)


@pytest.fixture(scope="module")
def c5(tmp_path_factory):
    d = tmp_path_factory.mktemp("config5")
    path = d / "model.bin"
    sp = config5_spec()
    print(f"[case] config 5: writing a {sp.n_layers}-layer checkpoint, vocab {sp.vocab_size}", flush=True)
    glm_model.write_synth_checkpoint(path, sp)
    ck = glm_model.Checkpoint(path)
    dec = glm_model.Decoder(ck, CTX + 2)
    assert dec.on_gpu(), "the whole forward runs on the GPU model"
    try:
        yield path, dec, d
    finally:
        dec.free()
        ck.close()
        os.remove(path)


def check_logits(got, want, what):
    assert_close(got, want, f"{what} logits")
    assert int(np.argmax(got)) == int(np.argmax(want)), f"{what}: argmax"


def test_zeroed_cache_at_position_4096_matches_glm(c5):
    path, dec, d = c5
    token, L, D, V = 4242, dec.L, dec.D, dec.V
    FP = C.POINTER(C.c_float)
    logits = np.zeros(V, np.float32)
    attn = np.zeros((L, D), np.float32)
    layer = np.zeros((L, D), np.float32)
    print(f"[case] config 5: GPU model at position {CTX} over its zeroed cache", flush=True)
    rc = dec.lib.glm_hip_model_forward(C.byref(dec.rt), C.byref(dec.st), token, CTX, 1, logits.ctypes.data_as(FP),
                                       attn.ctypes.data_as(FP), layer.ctypes.data_as(FP))
    assert rc == 0
    print("[case] config 5: glm.c's forward over a zeroed cache", flush=True)
    ref = ref_decode.reference_zero_cache(path, d / "zero", token, CTX, L, D, V)
    for l in range(L):
        assert_close(attn[l], ref["attn"][l], f"layer {l} attention")
        assert_close(layer[l], ref["layer"][l], f"layer {l} FFN")
    check_logits(logits, ref["logits"], "zeroed cache")


def test_after_a_4096_token_prefill_every_stage_matches_glm(c5):
    path, dec, d = c5
    L, D, V = dec.L, dec.D, dec.V
    rng = np.random.default_rng(50)
    prompt = rng.integers(3, V, CTX).astype(np.int32)
    print(f"[case] config 5: batched prefill of {CTX} tokens on the GPU model", flush=True)
    out = dec.prefill(prompt, 0)
    token = int(np.argmax(out))
    print(f"[case] config 5: token {token} at position {CTX} with dual checkpoints", flush=True)
    logits, attn, layer = dec.step(token, CTX, checkpoints=True)
    for l in range(L):
        comp, pe = dec.read_cache(l, 0, CTX, 512, 64)
        assert np.all(np.isfinite(comp)) and np.all(np.isfinite(pe))
        assert np.abs(comp).max() > 0, f"layer {l}: the cache holds the prompt"
        print(f"[case] config 5: layer {l} attention over {CTX + 1} positions", flush=True)
        want = ref_decode.reference_stage(path, d / f"attn{l}", 0, l, CTX, D, token=token,
                                          x_in=None if l == 0 else layer[l - 1], comp=comp, pe=pe)
        assert_close(attn[l], want, f"layer {l} attention")
        print(f"[case] config 5: layer {l} FFN", flush=True)
        want = ref_decode.reference_stage(path, d / f"ffn{l}", 1, l, CTX, D, x_in=attn[l])
        assert_close(layer[l], want, f"layer {l} FFN")
    print(f"[case] config 5: LM head over {V} rows", flush=True)
    want = ref_decode.reference_stage(path, d / "head", 2, 0, CTX, V, x_in=layer[L - 1])
    check_logits(logits, want, "after prefill")
