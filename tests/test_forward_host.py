"""glm.c's token forward in libglm_hip.so (glm_hip_forward_token, forward.c) on the host.

* A checkpoint without MoE layers (layer 0's MLA attention and dense FFN, final norm,
  LM head) runs entirely on the host: every position's x after attention, x after the
  FFN and the logits equal glm.c's own (oracle/_ref, infer.c:1767-1901) bit for bit,
  for both Q8_0 group sizes the exporter and the tiled form use.
* With MoE layers and no GPU backend, the forward fails (-1) instead of computing the
  MoE layers anywhere else.
* The checkpoint variants run on a copy: the state, its cache included, is unchanged.
* A position past the cache is an error, not an exit."""
import ctypes as C

import numpy as np
import pytest

import glm_model
import gmoe
import ref_decode


def spec(n_layers, gs=16, scale_mode=gmoe.SYNTH_SCALES_FP32, seed=9):
    return glm_model.CkptSpec(dim=256, hidden_dim=512, n_layers=n_layers, n_heads=4, n_kv_heads=4, vocab_size=300,
                              seq_len=64, rope_dim=16, q_lora_rank=64, kv_lora_rank=64, n_routed_experts=8,
                              n_experts_used=2, bos_id=1, eos_id=2, qk_nope_dim=32, v_head_dim=32, moe_ffn_dim=256,
                              group_size=gs, seed=seed, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                              bias_mode=gmoe.SYNTH_BIAS_NORMAL, scale_mode=scale_mode)


TOKENS = [1, 5, 17, 299, 42, 0, 17, 123]


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.skipif(not ref_decode.available(), reason="oracle/_ref not built (needs the reference sources)")
@pytest.mark.parametrize("gs,scale_mode", [(16, gmoe.SYNTH_SCALES_FP32), (32, gmoe.SYNTH_SCALES_FP16)])
def test_dense_model_matches_glm_bit_for_bit(tmp_path, gs, scale_mode):
    path = tmp_path / "dense.bin"
    glm_model.write_synth_checkpoint(path, spec(1, gs, scale_mode))
    cap = len(TOKENS) + 2
    ck = glm_model.Checkpoint(path)
    dec = glm_model.Decoder(ck, cap)
    try:
        assert dec.backend == glm_model.BACKEND_CPU
        ref = ref_decode.reference_decode(path, TOKENS, cap, dec.L, dec.D, dec.V, tmp_path / "ref")
        for pos, tok in enumerate(TOKENS):
            logits, attn, layer = dec.step(tok, pos, checkpoints=True)
            assert np.array_equal(bits(attn), bits(ref["attn"][pos])), f"pos {pos}: x after attention"
            assert np.array_equal(bits(layer), bits(ref["layer"][pos])), f"pos {pos}: x after the FFN"
            assert np.array_equal(bits(logits), bits(ref["logits"][pos])), f"pos {pos}: logits"
            assert dec.argmax() == int(np.argmax(ref["logits"][pos]))
    finally:
        dec.free()
        ck.close()


def test_moe_layers_need_the_gpu_backend(tmp_path):
    path = tmp_path / "moe.bin"
    glm_model.write_synth_checkpoint(path, spec(3))
    ck = glm_model.Checkpoint(path)
    lib = glm_model.forward_lib()
    st = glm_model.RunState()
    assert lib.glm_runstate_build(C.byref(st), C.byref(ck.rt), 4) == 0
    try:
        # no glm_backend_init(BACKEND_HIP): the MoE layers have nowhere to run
        assert lib.glm_hip_forward_token(C.byref(ck.rt), C.byref(st), 1, 0, 0) == -1
    finally:
        lib.glm_runstate_free(C.byref(st))
        ck.close()


def test_checkpoints_leave_the_state_alone_and_bad_positions_fail(tmp_path):
    path = tmp_path / "dense.bin"
    glm_model.write_synth_checkpoint(path, spec(1))
    ck = glm_model.Checkpoint(path)
    dec = glm_model.Decoder(ck, 3)
    try:
        c = ck.rt.cfg
        comp = np.ctypeslib.as_array(C.cast(dec.st.k_cache_comp, C.POINTER(C.c_float)), shape=(3 * c.kv_lora_rank,))
        dec.step(1, 0)
        cache0 = comp.copy()
        dec.step(5, 1, checkpoints=True)  # checkpoints on a copy, then the step itself
        assert not np.array_equal(comp, cache0), "the step writes position 1 of the cache"
        cache1, logits1 = comp.copy(), dec.logits()
        out = np.zeros((1, c.dim), np.float32)
        n = C.c_int()
        FP = C.POINTER(C.c_float)
        rc = dec.lib.glm_hip_forward_token_dual_checkpoints(C.byref(ck.rt), C.byref(dec.st), 7, 2, 0, None, 0, 0, None,
                                                           out.ctypes.data_as(FP), c.dim, 1, C.byref(n))
        assert rc == 0 and n.value == 1
        assert np.array_equal(comp, cache1), "dual checkpoints ran on a copy: the cache is as it was"
        assert np.array_equal(dec.logits(), logits1), "and so are the logits"
        # position 3 is past a cache of 3 positions: an error, the process goes on
        assert dec.lib.glm_hip_forward_token(C.byref(ck.rt), C.byref(dec.st), 7, 3, 0) == -1
    finally:
        dec.free()
        ck.close()


def test_prefill_without_the_gpu_model_is_the_token_loop(tmp_path):
    """glm_hip_prefill on a checkpoint the host forward runs: the same logits, x and cache
    as glm_hip_forward_token position by position; out-of-vocabulary tokens read as 0
    (infer.c:2220); a prefill past the cache fails and leaves the process running."""
    path = tmp_path / "dense.bin"
    glm_model.write_synth_checkpoint(path, spec(1, 32, gmoe.SYNTH_SCALES_FP16))
    ck = glm_model.Checkpoint(path)
    toks = [1, 5, 17, 299, 42, 0, 17, 123]
    a, b = glm_model.Decoder(ck, 12), glm_model.Decoder(ck, 12)
    try:
        c = ck.rt.cfg
        for pos, tok in enumerate(toks):
            a.step(tok, pos)
        got = b.prefill([1, 5, 17, 299, 42, -3, 17, 123])  # -3 is read as token 0
        assert np.array_equal(bits(got), bits(a.logits()))
        x = [np.ctypeslib.as_array(C.cast(d.st.x, C.POINTER(C.c_float)), shape=(c.dim,)) for d in (a, b)]
        assert np.array_equal(bits(x[0]), bits(x[1]))
        n = len(toks) * c.kv_lora_rank
        comp = [np.ctypeslib.as_array(C.cast(d.st.k_cache_comp, C.POINTER(C.c_float)), shape=(n,)) for d in (a, b)]
        assert np.array_equal(bits(comp[0]), bits(comp[1]))
        with pytest.raises(RuntimeError):
            b.prefill([3, 4, 5, 6, 7], pos0=len(toks))  # positions 8..12 of a 12-position cache
    finally:
        a.free()
        b.free()
        ck.close()
