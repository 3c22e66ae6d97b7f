"""glm.c's v4 checkpoint file (include/glm_ckpt.h): the synthetic writer and the reader.

* A written file opens with glm.c's own loader (runtime_open, infer.c:357-744, compiled
  from the reference sources into oracle/_ref): same header, and every tensor at the same
  offset as our reader finds it. The loader exits the process on a file it rejects, so it
  runs in a child process.
* The file's MoE tensors are the synthetic generator's for that seed, byte for byte, so a
  GPU test can check a loaded checkpoint against the oracle on regenerated layers.
* The reader refuses damaged files with an error, where glm.c's loader would exit."""
import ctypes as C
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import glm_model
import gmoe
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def small_spec(gs=16, scale_mode=gmoe.SYNTH_SCALES_FP32, seed=5, n_layers=3):
    return glm_model.CkptSpec(dim=256, hidden_dim=512, n_layers=n_layers, n_heads=4, n_kv_heads=4, vocab_size=300,
                              seq_len=64, rope_dim=16, q_lora_rank=64, kv_lora_rank=64, n_routed_experts=8,
                              n_experts_used=2, bos_id=1, eos_id=2, qk_nope_dim=32, v_head_dim=32, moe_ffn_dim=256,
                              group_size=gs, seed=seed, norm_mode=gmoe.SYNTH_NORM_RANDOM, bias_mode=gmoe.SYNTH_BIAS_NORMAL,
                              scale_mode=scale_mode)


REF_SCRIPT = r"""
import ctypes as C, json, sys
lib = C.CDLL(sys.argv[1])
lib.ref_ckpt_layout.argtypes = [C.c_char_p, C.POINTER(C.c_uint64), C.c_int, C.c_void_p]
lib.ref_ckpt_layout.restype = C.c_int
cfg = (C.c_uint8 * 256)()
out = (C.c_uint64 * 4096)()
n = lib.ref_ckpt_layout(sys.argv[2].encode(), out, 4096, cfg)
print(json.dumps({"layout": [int(v) for v in out[:n]], "cfg": list(cfg)}))
"""


def reference_layout(path):
    lib = oracle.PATHS["reference"]
    r = subprocess.run([sys.executable, "-c", REF_SCRIPT, lib, str(path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, f"glm.c's loader rejected the file: {r.stdout} {r.stderr}"
    return json.loads(r.stdout.strip().splitlines()[-1])


@pytest.mark.skipif(not oracle.available("reference"), reason="oracle/_ref not built (needs the reference sources)")
@pytest.mark.parametrize("gs,scale_mode", [(16, gmoe.SYNTH_SCALES_FP32), (32, gmoe.SYNTH_SCALES_FP16)])
def test_written_file_opens_with_glms_loader(tmp_path, gs, scale_mode):
    path = tmp_path / "synth.bin"
    glm_model.write_synth_checkpoint(path, small_spec(gs, scale_mode))
    ours = glm_model.Checkpoint(path)
    try:
        mine = ours.layout()
        cfg_mine = bytes(C.string_at(C.addressof(ours.rt.cfg), C.sizeof(glm_model.RuntimeConfig)))
        assert ours.rt.has_l0_ffn and ours.rt.has_l0_attn and ours.rt.has_all_attn
        assert ours.rt.has_moe_shared and ours.rt.has_moe_routed
    finally:
        ours.close()
    ref = reference_layout(path)
    assert bytes(ref["cfg"][:len(cfg_mine)]) == cfg_mine, "header as glm.c reads it"
    np.testing.assert_array_equal(np.array(ref["layout"], np.uint64), mine, err_msg="tensor offsets vs glm.c's loader")
    assert os.path.getsize(path) == ours_total(path)


def ours_total(path):
    ck = glm_model.Checkpoint(path)
    try:
        return int(ck.rt.cfg.total_bytes)
    finally:
        ck.close()


def test_moe_tensors_are_the_generators(tmp_path):
    sp = small_spec()
    path = tmp_path / "synth.bin"
    glm_model.write_synth_checkpoint(path, sp)
    shape = gmoe.Shape(dim=sp.dim, moe_ffn_dim=sp.moe_ffn_dim, n_routed_experts=sp.n_routed_experts,
                       n_experts_used=sp.n_experts_used, group_size=sp.group_size)
    ck = glm_model.Checkpoint(path)
    try:
        for l in range(1, sp.n_layers):
            hl = gmoe.HostLayer(shape, seed=sp.seed, layer=l, norm_mode=sp.norm_mode, bias_mode=sp.bias_mode,
                                scale_mode=sp.scale_mode)
            sh, ro = ck.rt.moe_layers[l], ck.rt.moe_routed_layers[l]
            for name in glm_model.SHARED_FIELDS:
                want = getattr(hl, name)
                got = np.ctypeslib.as_array(C.cast(getattr(sh, name), C.POINTER(np.ctypeslib.as_ctypes_type(want.dtype))),
                                            shape=want.shape)
                assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), f"layer {l} {name}"
            for name in glm_model.ROUTED_FIELDS:
                want = getattr(hl, name)
                got = np.ctypeslib.as_array(C.cast(getattr(ro, name), C.POINTER(np.ctypeslib.as_ctypes_type(want.dtype))),
                                            shape=want.shape)
                assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), f"layer {l} {name}"
    finally:
        ck.close()


def test_reader_refuses_damaged_files(tmp_path):
    path = tmp_path / "synth.bin"
    glm_model.write_synth_checkpoint(path, small_spec(n_layers=2))
    data = path.read_bytes()
    cases = {"short": data[:-1], "magic": b"\0\0\0\0" + data[4:], "tiny": data[:100],
             "group": data[:72] + (0).to_bytes(8, "little") + data[80:]}
    expect = {"short": "size mismatch", "magic": "magic", "tiny": "too small", "group": "group size"}
    for name, blob in cases.items():
        bad = tmp_path / f"{name}.bin"
        bad.write_bytes(blob)
        with pytest.raises(RuntimeError, match=expect[name]):
            glm_model.Checkpoint(bad)


def test_writer_refuses_shapes_the_group_size_does_not_divide(tmp_path):
    sp = small_spec()
    sp.q_lora_rank = 72  # not a multiple of 16
    with pytest.raises(RuntimeError, match="group size"):
        glm_model.write_synth_checkpoint(tmp_path / "bad.bin", sp)
