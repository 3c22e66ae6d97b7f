"""Batched prefill (glm_hip_prefill -> gmoe_model_prefill) against glm.c's own token-by-token
prompt loop (infer.c:2190-2220, compiled into oracle/_ref) on synthetic v4 checkpoints.

A prompt goes through the GPU model GLM_HIP_PREFILL_BATCH tokens at a time: each layer's
products over the whole batch in one launch, every token's cache entry written before the
attention reads it, each MoE layer one gmoe_forward over the batch (grouped expert GEMMs).
The last token's logits and final x are held to the FFN bar (max-abs 1e-2, rel-L2 1e-3)
against glm.c's at that position, with the same argmax. The decode that follows, one token
at a time on the cache the prefill wrote, must match glm.c's logits at every later
position, which checks every cache entry the prefill wrote (every attention layer reads all
of them). Batches of 1, 4 and 512 take the prompt whole, in ragged pieces
and one token at a time; a 150-token prompt in 64-token batches crosses attention's
32-position chunks inside a batch, and a 400-token prompt gives ranges of several tiles."""
import ctypes as C

import numpy as np
import pytest

import glm_model
import gmoe
import ref_decode
from conftest import assert_close
from test_gpu_forward import CASES, small

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not ref_decode.available(), reason="oracle/_ref not built (needs the reference sources)")]


def open_decoder(tmp_path, sp, cap):
    path = tmp_path / "model.bin"
    glm_model.write_synth_checkpoint(path, sp)
    ck = glm_model.Checkpoint(path)
    dec = glm_model.Decoder(ck, cap)
    assert dec.backend == glm_model.BACKEND_HIP and dec.on_gpu(), "the forward runs on the GPU model"
    return path, ck, dec


def final_x(dec):
    return np.ctypeslib.as_array(C.cast(dec.st.x, C.POINTER(C.c_float)), shape=(dec.D,)).copy()


def prefill_then_decode(tmp_path, sp, tokens, n_prompt, what):
    cap = len(tokens) + 1
    path, ck, dec = open_decoder(tmp_path, sp, cap)
    try:
        ref = ref_decode.reference_decode(path, tokens, cap, dec.L, dec.D, dec.V, tmp_path / "ref")
        print(f"[case] {what}: prefill of {n_prompt} tokens", flush=True)
        logits = dec.prefill(tokens[:n_prompt])
        last = n_prompt - 1
        assert_close(logits, ref["logits"][last], f"{what}: prefill logits")
        assert int(np.argmax(logits)) == int(np.argmax(ref["logits"][last])), f"{what}: prefill argmax"
        assert_close(final_x(dec), ref["layer"][last][dec.L - 1], f"{what}: x after the last layer")
        for pos in range(n_prompt, len(tokens)):
            print(f"[case] {what}: decode pos {pos}", flush=True)
            logits = dec.step(tokens[pos], pos)
            assert_close(logits, ref["logits"][pos], f"{what}: decode pos {pos} logits")
            assert int(np.argmax(logits)) == int(np.argmax(ref["logits"][pos])), f"{what}: pos {pos} argmax"
    finally:
        dec.free()
        ck.close()


@pytest.mark.parametrize("batch", ["1", "4", "512"])
@pytest.mark.parametrize("case", list(CASES))
def test_prefill_matches_glms_prompt_loop(tmp_path, monkeypatch, case, batch):
    monkeypatch.setenv("GLM_HIP_PREFILL_BATCH", batch)
    monkeypatch.delenv("GLM_HIP_HOST_ATTN", raising=False)
    sp = CASES[case]()
    tokens = [t % sp.vocab_size for t in [1, 5, 17, 299, 42, 0, 17, 123, 7, 250, 33, 9]]
    prefill_then_decode(tmp_path, sp, tokens, 10, f"{case} batch {batch}")


def test_long_prompt_in_batches_across_attention_chunks(tmp_path, monkeypatch):
    monkeypatch.setenv("GLM_HIP_PREFILL_BATCH", "64")
    monkeypatch.delenv("GLM_HIP_HOST_ATTN", raising=False)
    sp = small(32, gmoe.SYNTH_SCALES_FP16, n_layers=3, seed=24, seq_len=256)
    rng = np.random.default_rng(24)
    tokens = [1] + [int(t) for t in rng.integers(3, sp.vocab_size, 153)]
    prefill_then_decode(tmp_path, sp, tokens, 150, "long prompt batch 64")


def test_prefill_ranges_of_several_tiles(tmp_path, monkeypatch):
    """A 400-token prompt in one batch: a token's attention splits its positions into 8
    ranges, so past position 288 a range holds more than one 36-position tile and the
    next tile's loads are in flight while the current one is scored."""
    monkeypatch.setenv("GLM_HIP_PREFILL_BATCH", "512")
    monkeypatch.delenv("GLM_HIP_HOST_ATTN", raising=False)
    sp = small(32, gmoe.SYNTH_SCALES_FP16, n_layers=3, seed=27, seq_len=512)
    rng = np.random.default_rng(27)
    tokens = [1] + [int(t) for t in rng.integers(3, sp.vocab_size, 402)]
    prefill_then_decode(tmp_path, sp, tokens, 400, "400-token prompt")


def test_prefill_at_an_offset_and_past_the_cache(tmp_path, monkeypatch):
    """A second prefill continues at pos0 = the first's length; a prefill past the cache
    fails with -1 and the decoder goes on."""
    monkeypatch.setenv("GLM_HIP_PREFILL_BATCH", "8")
    monkeypatch.delenv("GLM_HIP_HOST_ATTN", raising=False)
    sp = CASES["gs32_tiled"]()
    tokens = [t % sp.vocab_size for t in [1, 5, 17, 299, 42, 0, 17, 123, 7, 250, 33, 9]]
    cap = len(tokens) + 1
    path, ck, dec = open_decoder(tmp_path, sp, cap)
    try:
        ref = ref_decode.reference_decode(path, tokens, cap, dec.L, dec.D, dec.V, tmp_path / "ref")
        dec.prefill(tokens[:5])
        logits = dec.prefill(tokens[5:11], pos0=5)
        assert_close(logits, ref["logits"][10], "second prefill logits")
        with pytest.raises(RuntimeError):
            dec.prefill(tokens[:4], pos0=cap - 2)
        logits = dec.step(tokens[11], 11)
        assert_close(logits, ref["logits"][11], "decode after the refused prefill")
    finally:
        dec.free()
        ck.close()


def test_merge_paths_agree_bit_for_bit(tmp_path, monkeypatch):
    """The batch attention's merge by one wave per (token, head) and k_attn_merge's block per
    64 columns (GMOE_ATTN_MERGE_WIDE=1) give the same bits: the prefill's logits and final x
    over a 400-token prompt in one batch (eight position chunks per token)."""
    monkeypatch.setenv("GLM_HIP_PREFILL_BATCH", "512")
    monkeypatch.delenv("GLM_HIP_HOST_ATTN", raising=False)
    sp = small(32, gmoe.SYNTH_SCALES_FP16, n_layers=3, seed=28, seq_len=512)
    rng = np.random.default_rng(28)
    tokens = [1] + [int(t) for t in rng.integers(3, sp.vocab_size, 399)]
    out = {}
    for wide in ("0", "1"):
        monkeypatch.setenv("GMOE_ATTN_MERGE_WIDE", wide)
        d = tmp_path / f"wide{wide}"
        d.mkdir()
        _, ck, dec = open_decoder(d, sp, len(tokens) + 1)
        try:
            print(f"[case] merge paths: GMOE_ATTN_MERGE_WIDE={wide}", flush=True)
            logits = dec.prefill(tokens)
            out[wide] = (logits.copy(), final_x(dec))
        finally:
            dec.free()
            ck.close()
    assert np.array_equal(out["0"][0].view(np.uint32), out["1"][0].view(np.uint32)), "prefill logits"
    assert np.array_equal(out["0"][1].view(np.uint32), out["1"][1].view(np.uint32)), "final x"
