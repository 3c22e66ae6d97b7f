"""The drop-in boundary on the GPU: glm.c's backend interface (backend.h:7-13) with
BACKEND_HIP, driven exactly as glm.c would drive it.

A synthetic Runtime/RunState (include/glm_model.h, filled as infer.c:640-743 and
855-862 fill them) goes to glm_backend_init(BACKEND_HIP), which uploads every MoE layer;
then glm_backend_try_hip_moe runs layers 1..L-1 on st in place, the hook at the top of
apply_moe_shared_ffn_layer. After each layer the RunState must hold what
infer.c:1098-1214 leaves there: x, xn, moe_router, moe_topk_idx, moe_topk_w, xb and
moe_out_acc, checked against the oracle on the same input."""
import numpy as np
import pytest

import gmoe
import glm_model
import oracle
from conftest import assert_close

pytestmark = pytest.mark.gpu


def run_backend_layers(shape, layers, x0, env=None, monkeypatch=None):
    model = glm_model.GlmModel(shape, layers)
    if env:
        for k, v in env.items():
            monkeypatch.setenv(k, v)
    print(f"[case] glm_backend_init(BACKEND_HIP) D={shape.D} E={shape.E} layers={len(layers)}", flush=True)
    assert model.init() == glm_model.BACKEND_HIP
    return model


def test_backend_runs_each_moe_layer_on_the_run_state(dkernel):
    shape = gmoe.GLM47_FLASH
    layers = [gmoe.HostLayer(shape, seed=21, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM) for l in (1, 2, 3)]
    model = run_backend_layers(shape, layers, None)
    orc = oracle.Oracle("port")
    try:
        model.buf["x"][:] = gmoe.activations(21, 0, 1, shape.D)[0]
        for l in range(1, len(layers) + 1):
            x_in = model.buf["x"].copy()
            want = orc.layer(shape, layers[l - 1], x_in[None, :])
            print(f"[case] glm_backend_try_hip_moe layer {l}", flush=True)
            assert model.try_moe(l) == 0
            b = model.buf
            np.testing.assert_array_equal(b["moe_topk_idx"], want["topk_idx"][0], err_msg=f"layer {l} moe_topk_idx")
            assert np.array_equal(b["xn"].view(np.uint32), want["xn"][0].view(np.uint32)), f"layer {l} xn"
            assert_close(b["moe_router"], want["router_prob"][0], f"layer {l} moe_router", max_abs=1e-5, rel_l2=1e-5)
            assert_close(b["moe_topk_w"], want["topk_w"][0], f"layer {l} moe_topk_w", max_abs=1e-5, rel_l2=1e-5)
            assert_close(b["xb"], want["shared_out"][0], f"layer {l} xb")
            assert_close(b["moe_out_acc"], want["routed_out"][0], f"layer {l} moe_out_acc")
            assert_close(b["x"], want["x_out"][0], f"layer {l} x")
        # a layer index without a MoE block is a no-op that succeeds, as infer.c:1088-1092
        x_before = model.buf["x"].copy()
        assert model.try_moe(0) == 0
        assert np.array_equal(model.buf["x"], x_before)
    finally:
        model.free()


def test_backend_declines_a_failed_layer_and_keeps_x(monkeypatch, dkernel):
    """A GPU layer that fails returns -1 so glm.c runs the layer on the CPU, and that
    needs st->x as it was: the forced timeout (GMOE_SPIN_LIMIT=0) must leave it intact."""
    shape = gmoe.Shape(dim=256, moe_ffn_dim=256, n_routed_experts=16, n_experts_used=4)
    layers = [gmoe.HostLayer(shape, seed=22, layer=1)]
    model = run_backend_layers(shape, layers, None, env={"GMOE_SPIN_LIMIT": "0"}, monkeypatch=monkeypatch)
    try:
        model.buf["x"][:] = gmoe.activations(22, 0, 1, shape.D)[0]
        before = model.buf["x"].copy()
        print("[case] glm_backend_try_hip_moe with every wait starved", flush=True)
        assert model.try_moe(1) == -1
        assert np.array_equal(model.buf["x"].view(np.uint32), before.view(np.uint32))
    finally:
        model.free()
