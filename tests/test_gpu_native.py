"""Checkpoints in glm.c's own Q8_0 form on the GPU: group size 16 as the exporter writes
it (glm47_flash_export.py:36), fp32 scales that fp16 cannot hold (max|w|/127 there,
glm47_flash_export.py:157-169; random fp32 here), and other group sizes (infer.c:380-385,
646 take any). Group size 16 runs in two device forms: GMOE_Q8_TILED16 (what AUTO picks:
the tiled q planes with the fp32 scales kept as they are, on the relay decode kernel and
the grouped GEMMs) and GMOE_Q8_NATIVE (glm.c's layout, native kernels); the tests name the
kernels that ran. Each case runs against the oracle, which follows infer.c:765-786 for any
group size. Bar as elsewhere: top-k exact, xn bit for bit, router probabilities and
weights within 1e-5, outputs within max-abs 1e-2 and rel-L2 1e-3."""
import numpy as np
import pytest

import gmoe
import glm_model
import oracle
from conftest import assert_close

pytestmark = pytest.mark.gpu

GLM16 = gmoe.Shape(group_size=16)
SMALL64 = gmoe.Shape(dim=512, moe_ffn_dim=256, n_routed_experts=16, n_experts_used=4, group_size=64)


def check(want, got, st, what):
    np.testing.assert_array_equal(st["topk_idx"], want["topk_idx"], err_msg=f"{what}: top-k")
    assert np.array_equal(st["xn"].view(np.uint32), want["xn"].view(np.uint32)), f"{what}: xn"
    assert_close(st["router_prob"], want["router_prob"], f"{what}: router_prob", max_abs=1e-5, rel_l2=1e-5)
    assert_close(st["topk_w"], want["topk_w"], f"{what}: topk_w", max_abs=1e-5, rel_l2=1e-5)
    assert_close(st["shared_out"], want["shared_out"], f"{what}: shared_out")
    assert_close(st["routed_out"], want["routed_out"], f"{what}: routed_out")
    assert_close(got, want["x_out"], f"{what}: x_out")


GS16_FORMS = [pytest.param(gmoe.GMOE_Q8_AUTO, id="tiled16"), pytest.param(gmoe.GMOE_Q8_NATIVE, id="native")]


def expect_kernels(ctx, q8_form, T):
    """The form AUTO resolved to at group size 16, and the kernels the profiled calls ran."""
    ran = ctx.profile_read()
    if q8_form == gmoe.GMOE_Q8_NATIVE:
        assert ctx.stats()["q8_form"] == gmoe.GMOE_Q8_NATIVE
        assert "k_moe_relay" not in ran and "k_act_split" not in ran, ran
    else:
        assert ctx.stats()["q8_form"] == gmoe.GMOE_Q8_TILED16
        if T == 1:
            assert "k_moe_relay" in ran and "gate_up" not in ran, ran
        else:
            assert "k_act_split" in ran and "gate_up" in ran and "k_moe_relay" not in ran, ran  # k_group_gu


def run(shape, seed, T, q8_form=gmoe.GMOE_Q8_AUTO, flags=0, n_layers=1):
    layers = [gmoe.HostLayer(shape, seed=seed, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                             scale_mode=gmoe.SYNTH_SCALES_FP32) for l in range(1, n_layers + 1)]
    ctx = gmoe.Context(shape, n_layers=n_layers + 1, max_tokens=T, q8_form=q8_form)
    orc = oracle.Oracle("port")
    try:
        for l, hl in enumerate(layers, start=1):
            ctx.upload(l, hl)
        ctx.profile(True)
        x = gmoe.activations(seed, 7, T, shape.D)
        for l, hl in enumerate(layers, start=1):
            print(f"[case] gs={shape.gs} form={q8_form} D={shape.D} E={shape.E} T={T} layer {l} flags={flags}", flush=True)
            want = orc.layer(shape, hl, x, disable_routed=bool(flags & gmoe.GMOE_FLAG_NO_ROUTED))
            got, st = gmoe.forward_host(ctx, l, x, flags=flags)
            check(want, got, st, f"gs={shape.gs} T={T} layer {l}")
            x = got
        return ctx.profile_read(), ctx.stats()
    finally:
        ctx.close()


@pytest.mark.parametrize("q8_form", GS16_FORMS)
def test_gs16_fp32_scales_decode(q8_form):
    ran, stats = run(GLM16, seed=41, T=1, n_layers=3, q8_form=q8_form)
    if q8_form == gmoe.GMOE_Q8_AUTO:
        assert stats["q8_form"] == gmoe.GMOE_Q8_TILED16 and ran["k_moe_relay"][0] == 3, (stats, ran)
    else:
        assert stats["q8_form"] == gmoe.GMOE_Q8_NATIVE and "k_moe_relay" not in ran, (stats, ran)


@pytest.mark.parametrize("q8_form", GS16_FORMS)
def test_gs16_fp32_scales_batch_and_lists(q8_form):
    shape, T = GLM16, 6
    hl = gmoe.HostLayer(shape, seed=42, layer=1, scale_mode=gmoe.SYNTH_SCALES_FP32)
    ctx = gmoe.Context(shape, n_layers=2, max_tokens=T, q8_form=q8_form)
    try:
        ctx.upload(1, hl)
        ctx.profile(True)
        x = gmoe.activations(42, 1, T, shape.D)
        print(f"[case] gs=16 form={q8_form} T={T} with per-expert lists", flush=True)
        want = oracle.Oracle("port").layer(shape, hl, x)
        got, st = gmoe.forward_host(ctx, 1, x)
        check(want, got, st, "gs=16 batch")
        expect_kernels(ctx, q8_form, T)
        # per-expert lists: the ascending tokens of each expert, a brute-force grouping
        offs, toks = [0], []
        for e in range(shape.E):
            toks += [t for t in range(T) if e in want["topk_idx"][t]]
            offs.append(len(toks))
        np.testing.assert_array_equal(st["expert_offsets"], np.array(offs, np.int32), err_msg="per-expert offsets")
        np.testing.assert_array_equal(st["expert_tokens"], np.array(toks, np.int32), err_msg="per-expert token lists")
    finally:
        ctx.close()


def test_gs16_routed_experts_off():
    run(GLM16, seed=43, T=2, flags=gmoe.GMOE_FLAG_NO_ROUTED)
    run(GLM16, seed=43, T=1, flags=gmoe.GMOE_FLAG_NO_ROUTED)


@pytest.mark.parametrize("T", [128, 37])
def test_gs16_prefill_batch(T):
    """A prefill-sized batch at group size 16 (every expert's list several tiles long at
    T=128; ragged tiles at T=37) on the grouped GEMMs, against the oracle."""
    shape = GLM16
    hl = gmoe.HostLayer(shape, seed=47, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM, scale_mode=gmoe.SYNTH_SCALES_FP32)
    ctx = gmoe.Context(shape, n_layers=2, max_tokens=T)
    try:
        ctx.upload(1, hl)
        ctx.profile(True)
        x = gmoe.activations(47, 1, T, shape.D)
        print(f"[case] gs=16 tiled16 prefill T={T}", flush=True)
        want = oracle.Oracle("port").layer(shape, hl, x)
        got, st = gmoe.forward_host(ctx, 1, x)
        check(want, got, st, f"gs=16 prefill T={T}")
        expect_kernels(ctx, gmoe.GMOE_Q8_AUTO, T)
    finally:
        ctx.close()


def test_gs16_layers_in_one_launch():
    """Three gs=16 layers in one k_moe_relay launch (gmoe_forward_layers), against the
    oracle layer by layer, and the same as three one-layer launches bit for bit."""
    shape, n = GLM16, 3
    layers = [gmoe.HostLayer(shape, seed=48, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                             scale_mode=gmoe.SYNTH_SCALES_FP32) for l in range(1, n + 1)]
    ctx = gmoe.Context(shape, n_layers=n + 1, max_tokens=1)
    orc = oracle.Oracle("port")
    try:
        for l, hl in enumerate(layers, start=1):
            ctx.upload(l, hl)
        assert ctx.stats()["q8_form"] == gmoe.GMOE_Q8_TILED16
        x = gmoe.activations(48, 3, 1, shape.D)
        want = x
        for l, hl in enumerate(layers, start=1):
            want = orc.layer(shape, hl, want)["x_out"]
        print("[case] gs=16 tiled16, 3 layers in one launch", flush=True)
        d_in = gmoe.DeviceArray.from_numpy(x)
        d_out = gmoe.DeviceArray(x.nbytes)
        ctx.forward_layers(1, n, 1, d_in.ptr, d_out.ptr)
        got = d_out.download((1, shape.D), np.float32)
        assert_close(got, want, "3-layer x_out")
        one = x
        for l in range(1, n + 1):
            one, _ = gmoe.forward_host(ctx, l, one)
        assert np.array_equal(got.view(np.uint32), one.view(np.uint32)), "one launch vs per-layer launches"
    finally:
        ctx.close()


def test_tiled16_refused_where_the_relay_kernel_cannot_run(monkeypatch):
    """GMOE_Q8_TILED16 runs on k_moe_relay only: with it switched off the context is
    refused with a message; AUTO then keeps group size 16 in the native form."""
    monkeypatch.setenv("GMOE_DECODE_KERNEL", "0")
    with pytest.raises(RuntimeError, match="TILED16"):
        gmoe.Context(GLM16, n_layers=2, max_tokens=1, q8_form=gmoe.GMOE_Q8_TILED16)
    ctx = gmoe.Context(GLM16, n_layers=2, max_tokens=1)
    try:
        assert ctx.stats()["q8_form"] == gmoe.GMOE_Q8_NATIVE
    finally:
        ctx.close()


def test_gs64_small_shape():
    run(SMALL64, seed=44, T=3, n_layers=2)


def test_gs32_fp32_scales_need_the_native_form():
    """fp32 scales at group size 32: the tiled form refuses them (GMOE_ERR_SCALE); the
    native form computes them as glm.c does."""
    shape = gmoe.GLM47_FLASH
    hl = gmoe.HostLayer(shape, seed=45, layer=1, scale_mode=gmoe.SYNTH_SCALES_FP32)
    ctx = gmoe.Context(shape, n_layers=2, max_tokens=1)
    try:
        print("[case] tiled form refuses fp32 scales", flush=True)
        rc = ctx.lib.gmoe_upload_layer(ctx.h, 1, gmoe.C.byref(hl.weights()))
        assert rc == -4, rc
        assert "fp16" in gmoe.last_error()
    finally:
        ctx.close()
    run(shape, seed=45, T=1, q8_form=gmoe.GMOE_Q8_NATIVE)


@pytest.mark.parametrize("shape", [GLM16, gmoe.GLM47_FLASH], ids=["gs16", "gs32_fp32"])
def test_backend_takes_exporter_checkpoints(shape):
    """glm_backend_init(BACKEND_HIP) on a checkpoint with fp32 scales: at group size 16 the
    context is native from the start; at 32 the tiled upload fails on the scales and the
    backend re-creates the context in glm.c's layout. Either way the RunState matches."""
    layers = [gmoe.HostLayer(shape, seed=46, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                             scale_mode=gmoe.SYNTH_SCALES_FP32) for l in (1, 2)]
    model = glm_model.GlmModel(shape, layers)
    print(f"[case] backend with fp32 scales, gs={shape.gs}", flush=True)
    assert model.init() == glm_model.BACKEND_HIP
    orc = oracle.Oracle("port")
    try:
        model.buf["x"][:] = gmoe.activations(46, 0, 1, shape.D)[0]
        for l in (1, 2):
            x_in = model.buf["x"].copy()
            want = orc.layer(shape, layers[l - 1], x_in[None, :])
            assert model.try_moe(l) == 0
            b = model.buf
            np.testing.assert_array_equal(b["moe_topk_idx"], want["topk_idx"][0], err_msg=f"layer {l} moe_topk_idx")
            assert_close(b["xb"], want["shared_out"][0], f"layer {l} xb")
            assert_close(b["moe_out_acc"], want["routed_out"][0], f"layer {l} moe_out_acc")
            assert_close(b["x"], want["x_out"][0], f"layer {l} x")
    finally:
        model.free()


@pytest.mark.parametrize("gs,scale_mode", [(16, gmoe.SYNTH_SCALES_FP32), (32, gmoe.SYNTH_SCALES_FP16)],
                         ids=["gs16", "gs32_tiled"])
def test_backend_runs_a_checkpoint_file(tmp_path, gs, scale_mode):
    """A v4 .bin written by glm_ckpt_write_synth and mapped by glm_ckpt_open (the Runtime
    glm.c's runtime_open would fill) goes to glm_backend_init(BACKEND_HIP); each MoE layer
    then runs on the GPU against the oracle on the same layer, regenerated from the seed."""
    spec = glm_model.CkptSpec(dim=512, hidden_dim=1024, n_layers=3, n_heads=4, n_kv_heads=4, vocab_size=200,
                              seq_len=64, rope_dim=16, q_lora_rank=128, kv_lora_rank=64, n_routed_experts=16,
                              n_experts_used=4, bos_id=1, eos_id=2, qk_nope_dim=32, v_head_dim=32, moe_ffn_dim=256,
                              group_size=gs, seed=61, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                              bias_mode=gmoe.SYNTH_BIAS_NORMAL, scale_mode=scale_mode)
    path = tmp_path / "model.bin"
    glm_model.write_synth_checkpoint(path, spec)
    shape = gmoe.Shape(dim=spec.dim, moe_ffn_dim=spec.moe_ffn_dim, n_routed_experts=spec.n_routed_experts,
                       n_experts_used=spec.n_experts_used, group_size=gs)
    ck = glm_model.Checkpoint(path)
    model = glm_model.GlmModel(shape, checkpoint=ck)
    print(f"[case] backend on a checkpoint file, gs={gs}", flush=True)
    assert model.init() == glm_model.BACKEND_HIP
    orc = oracle.Oracle("port")
    try:
        model.buf["x"][:] = gmoe.activations(61, 0, 1, shape.D)[0]
        for l in range(1, spec.n_layers):
            hl = gmoe.HostLayer(shape, seed=spec.seed, layer=l, norm_mode=spec.norm_mode, scale_mode=scale_mode)
            x_in = model.buf["x"].copy()
            want = orc.layer(shape, hl, x_in[None, :])
            assert model.try_moe(l) == 0
            b = model.buf
            np.testing.assert_array_equal(b["moe_topk_idx"], want["topk_idx"][0], err_msg=f"layer {l} moe_topk_idx")
            assert np.array_equal(b["xn"].view(np.uint32), want["xn"][0].view(np.uint32)), f"layer {l} xn"
            assert_close(b["xb"], want["shared_out"][0], f"layer {l} xb")
            assert_close(b["moe_out_acc"], want["routed_out"][0], f"layer {l} moe_out_acc")
            assert_close(b["x"], want["x_out"][0], f"layer {l} x")
    finally:
        model.free()
        ck.close()


@pytest.mark.parametrize("shape", [
    gmoe.Shape(dim=1024, moe_ffn_dim=512, n_routed_experts=64, n_experts_used=4, group_size=16),
    gmoe.Shape(dim=2048, moe_ffn_dim=512, n_routed_experts=128, n_experts_used=6, group_size=16),
    gmoe.Shape(dim=512, moe_ffn_dim=512, n_routed_experts=256, n_experts_used=8, group_size=16),
], ids=["d1024_e64", "d2048_e128", "d512_e256"])
@pytest.mark.parametrize("T", [1, 9])
def test_gs16_tiled_other_shapes(shape, T):
    """The group-size-16 tiled form beyond the GLM shape: narrower rows (the relay kernel's
    shared-memory scale path), 128 and 256 experts (its wider selections), on the relay
    kernel at T=1 and the grouped GEMMs at T=9."""
    ran, stats = run(shape, seed=49, T=T, n_layers=2)
    assert stats["q8_form"] == gmoe.GMOE_Q8_TILED16, stats
    if T == 1:
        assert "k_moe_relay" in ran, ran
    else:
        assert "k_act_split" in ran and "gate_up" in ran, ran
