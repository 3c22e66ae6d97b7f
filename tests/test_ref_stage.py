"""The stage-by-stage form of glm.c's forward that the full-size GPU checks use
(ref_stage, ref_forward_zero_cache in oracle/ref_harness.c): chained on its own outputs at
position 0, the stages give glm.c's dual checkpoints and logits bit for bit, and the
zeroed-cache forward at position 0 is glm.c's forward of a fresh state."""
import numpy as np
import pytest

import app_runner
import glm_model
import ref_decode

pytestmark = pytest.mark.skipif(not ref_decode.available(), reason="oracle/_ref not built (needs the reference sources)")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_stages_chain_into_glms_forward(tmp_path):
    sp = app_runner.small_spec(seed=8, n_layers=3, seq_len=16)
    path = tmp_path / "model.bin"
    glm_model.write_synth_checkpoint(path, sp)
    token, L, D, V = 77, sp.n_layers, sp.dim, sp.vocab_size
    ref = ref_decode.reference_decode(path, [token], 2, L, D, V, tmp_path / "ref")
    x = None
    for l in range(L):
        x = ref_decode.reference_stage(path, tmp_path / f"a{l}", 0, l, 0, D, token=token, x_in=x)
        assert np.array_equal(bits(x), bits(ref["attn"][0][l])), f"layer {l} attention"
        x = ref_decode.reference_stage(path, tmp_path / f"f{l}", 1, l, 0, D, x_in=x)
        assert np.array_equal(bits(x), bits(ref["layer"][0][l])), f"layer {l} FFN"
    logits = ref_decode.reference_stage(path, tmp_path / "h", 2, 0, 0, V, x_in=x)
    assert np.array_equal(bits(logits), bits(ref["logits"][0]))
    z = ref_decode.reference_zero_cache(path, tmp_path / "z", token, 0, L, D, V)
    assert np.array_equal(bits(z["logits"]), bits(ref["logits"][0]))
    assert np.array_equal(bits(z["layer"]), bits(ref["layer"][0]))
