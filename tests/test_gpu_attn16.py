"""The batch attention on fp16 matrix cores with split operands (k_attn_tile16) against the
fp32 MFMA kernel it replaces (GMOE_ATTN_TILE_FP32=1), on the same model and prompt.

Both take the same tiles, chunks and partial-result slots; k_attn_tile16 forms each product
as hi.hi + hi.lo + lo.hi of fp16 halves (~22 bits of each operand) with power-of-two
exponents per query row and per cached row, so its results differ from fp32 products in
the last few bits only. The logits after a batched prefill are held to a tight bar against
the fp32 kernel's (max-abs 2e-4, rel-L2 2e-5: ~100x below the bar against glm.c, which
test_gpu_prefill.py and test_gpu_config5.py apply to the default kernel), with the same
argmax. Shapes: a small one (kv 64 + rope 16 = 80 columns: the last 32-column step is
padded with zeros) and glm.c's attention ranks (kv 512 + rope 64), 4 and 20 heads. Prompts:
300 tokens in one batch (five 64-token query tiles, several position chunks), then 200 more
at position 300 over that cache (chunks that span both batches, causal masks inside); then
a decode token with GMOE_MODEL_KEEP_CACHE at position 250 (its fp32 entries written, then
restored; the split form, which decode steps do not write, must be left as the prefill
wrote it), three tokens decoded one at a time (fp32 entries only: the next prefill converts
them with k_spl_fill before its attention) and 8 more tokens in a batch over all of them."""
import os

import numpy as np
import pytest

import gmoe
from conftest import assert_close

pytestmark = pytest.mark.gpu

KEEP_CACHE = 1  # GMOE_MODEL_KEEP_CACHE, include/gmoe_model.h


def small():
    return dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, vocab_size=300, q_lora_rank=64, kv_lora_rank=64,
                rope_dim=16, qk_nope_dim=32, head_k_dim=48, v_head_dim=32, group_size=32, cache_cap=512,
                attn_layers=2, has_l0_ffn=1, max_batch=300)


def glm_ranks(heads):
    return dict(dim=2048, hidden_dim=1024, n_layers=2, n_heads=heads, vocab_size=300, q_lora_rank=256,
                kv_lora_rank=512, rope_dim=64, qk_nope_dim=192, head_k_dim=256, v_head_dim=256, group_size=32,
                cache_cap=512, attn_layers=2, has_l0_ffn=1, max_batch=300)


CASES = {"small": small, "h4": lambda: glm_ranks(4), "h20": lambda: glm_ranks(20)}


def run(model, tokens, pos0, fp32):
    old = os.environ.get("GMOE_ATTN_TILE_FP32")
    try:
        if fp32:
            os.environ["GMOE_ATTN_TILE_FP32"] = "1"
        else:
            os.environ.pop("GMOE_ATTN_TILE_FP32", None)
        return model.prefill(tokens, pos0).copy()
    finally:
        if old is None:
            os.environ.pop("GMOE_ATTN_TILE_FP32", None)
        else:
            os.environ["GMOE_ATTN_TILE_FP32"] = old


@pytest.mark.parametrize("name", list(CASES))
def test_split_fp16_attention_matches_fp32(name):
    cfg = CASES[name]()
    g, attn = gmoe.synth_model_weights(cfg, 17)
    model = gmoe.Model(cfg)
    try:
        model.upload(g)
        for l, a in enumerate(attn):
            model.upload_attn(l, a)
        rng = np.random.default_rng(5)
        first = rng.integers(0, cfg["vocab_size"], 300).astype(np.int32)
        second = rng.integers(0, cfg["vocab_size"], 200).astype(np.int32)
        def check(what, toks, pos0):
            print(f"[case] {name}: {what}", flush=True)
            want = run(model, toks, pos0, fp32=True)
            got = run(model, toks, pos0, fp32=False)
            assert np.isfinite(got).all()
            assert_close(got, want, f"{name} {what}: logits", max_abs=2e-4, rel_l2=2e-5)
            assert int(np.argmax(got)) == int(np.argmax(want)), f"{name} {what}: argmax"

        check("300 tokens at 0", first, 0)
        check("200 tokens at 300", second, 300)
        # a kept decode token overwrites position 250's fp32 entries and restores them; tokens
        # decoded one at a time write fp32 entries only; a batch then reads both in split form
        model.forward_token(7, 250, flags=KEEP_CACHE)
        for pos in range(500, 503):
            model.forward_token(int(rng.integers(0, cfg["vocab_size"])), pos)
        check("8 tokens at 503 after kept and decoded tokens", rng.integers(0, cfg["vocab_size"], 8).astype(np.int32), 503)
    finally:
        model.close()
