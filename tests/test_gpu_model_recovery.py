"""The whole-model decode (gmoe_model_forward_token) after a token that could not run.

A token whose MoE layer is not uploaded to the model's context must fail before the
decode kernel's workspace is reset for the token's layers: a reset followed by an early
return would leave workspace layers whose parity was flipped but never written, and the
next token's flip would then make their stale words look current (silently wrong x, not
a timeout). After the missing layer is uploaded, the next tokens must equal, bit for bit,
those of a model that never failed."""
import numpy as np
import pytest

import gmoe

pytestmark = pytest.mark.gpu

CFG = dict(dim=256, hidden_dim=512, n_layers=4, n_heads=4, vocab_size=300, q_lora_rank=64, kv_lora_rank=64,
           rope_dim=16, qk_nope_dim=32, head_k_dim=48, v_head_dim=32, group_size=32, cache_cap=8, attn_layers=4,
           has_l0_ffn=1, max_batch=1)
SHAPE = gmoe.Shape(dim=256, moe_ffn_dim=256, n_routed_experts=8, n_experts_used=2)
TOKENS = [5, 17, 299, 42]


def build(g, attn, moe, upload):
    ctx = gmoe.Context(SHAPE, n_layers=CFG["n_layers"], max_tokens=1)
    for l in upload:
        ctx.upload(l, moe[l])
    model = gmoe.Model(CFG)
    model.upload(g)
    for l, a in enumerate(attn):
        model.upload_attn(l, a)
    model.set_moe(ctx, range(1, CFG["n_layers"]))
    return ctx, model


def test_token_with_a_missing_moe_layer_fails_cleanly_and_decode_resumes():
    g, attn = gmoe.synth_model_weights(CFG, 31)
    moe = {l: gmoe.HostLayer(SHAPE, seed=31, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM) for l in (1, 2, 3)}
    ctx_r, ref = build(g, attn, moe, (1, 2, 3))
    ctx, model = build(g, attn, moe, (1, 3))  # layer 2 missing
    try:
        print("[case] token with MoE layer 2 not uploaded", flush=True)
        with pytest.raises(RuntimeError, match="MoE layer 2 is not uploaded"):
            model.forward_token(TOKENS[0], 0)
        ctx.upload(2, moe[2])
        for pos, tok in enumerate(TOKENS):
            print(f"[case] resumed decode pos {pos}", flush=True)
            want = ref.forward_token(tok, pos).copy()
            got = model.forward_token(tok, pos).copy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"pos {pos}: logits differ"
    finally:
        model.close()
        ctx.close()
        ref.close()
        ctx_r.close()
