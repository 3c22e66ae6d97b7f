"""The persistent decode kernel (T=1 through a run of MoE layers in one launch).

Checks: one launch over n layers equals n single-layer launches bit for bit;
every layer's routing equals the oracle's on that layer's own input, and its
output is within the parity bar; the whole stack stays within the bar of the
oracle's stack (the decode loop of infer.c:1818-1860, MoE half)."""
import numpy as np
import pytest

import gmoe
import oracle
from conftest import DECODE_KERNEL_NAMES, assert_close, assert_decode_kernel, decode_kernel, launched

pytestmark = pytest.mark.gpu

N_LAYERS = 6


@pytest.fixture(scope="module", params=list(DECODE_KERNEL_NAMES))
def stack(request):
    shape = gmoe.GLM47_FLASH
    layers = [gmoe.HostLayer(shape, seed=11, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM) for l in range(1, N_LAYERS + 1)]
    with decode_kernel(request.param):
        ctx = gmoe.Context(shape, n_layers=N_LAYERS + 1, max_tokens=1)
    ctx.kind = request.param
    for l, hl in enumerate(layers, start=1):
        ctx.upload(l, hl)
    yield shape, layers, ctx
    ctx.close()


def test_one_launch_equals_layer_by_layer(stack):
    shape, layers, ctx = stack
    x0 = gmoe.activations(11, 1, 1, shape.D)
    print(f"[case] stack {N_LAYERS} layers, one launch vs per-layer ({ctx.kind})", flush=True)
    d_in = gmoe.DeviceArray.from_numpy(x0)
    d_out = gmoe.DeviceArray(x0.nbytes)
    ran = launched(ctx, lambda: ctx.forward_layers(1, N_LAYERS, 1, d_in.ptr, d_out.ptr))
    assert_decode_kernel(ran, ctx.kind)
    x_one = d_out.download((1, shape.D), np.float32)
    topk_one = [ctx.read_topk(l, 1)[0] for l in range(1, N_LAYERS + 1)]
    x = x0.copy()
    for l in range(1, N_LAYERS + 1):
        x, st = gmoe.forward_host(ctx, l, x)
        np.testing.assert_array_equal(st["topk_idx"], topk_one[l - 1], err_msg=f"layer {l} routing")
    assert np.array_equal(x.view(np.uint32), x_one.view(np.uint32)), "one launch differs from per-layer launches"


def test_each_layer_against_oracle(stack):
    shape, layers, ctx = stack
    x = gmoe.activations(11, 2, 1, shape.D)
    orc = oracle.Oracle("port")
    for l in range(1, N_LAYERS + 1):
        print(f"[case] stack layer {l} vs oracle", flush=True)
        want = orc.layer(shape, layers[l - 1], x)
        got, st = gmoe.forward_host(ctx, l, x)
        np.testing.assert_array_equal(st["topk_idx"], want["topk_idx"], err_msg=f"layer {l} routing")
        assert np.array_equal(st["xn"].view(np.uint32), want["xn"].view(np.uint32)), f"layer {l} xn"
        assert_close(st["topk_w"], want["topk_w"], f"layer {l} topk_w", max_abs=1e-5, rel_l2=1e-5)
        assert_close(st["shared_out"], want["shared_out"], f"layer {l} shared_out")
        assert_close(st["routed_out"], want["routed_out"], f"layer {l} routed_out")
        assert_close(got, want["x_out"], f"layer {l} x_out")
        x = got  # next layer starts from the GPU's own output


def test_stack_against_oracle_stack(stack):
    shape, layers, ctx = stack
    x0 = gmoe.activations(11, 3, 1, shape.D)
    print(f"[case] stack {N_LAYERS} layers vs oracle stack", flush=True)
    want_x, want_topk = oracle.Oracle("port").stack(shape, layers, x0)
    d_in = gmoe.DeviceArray.from_numpy(x0)
    ctx.forward_layers(1, N_LAYERS, 1, d_in.ptr, d_in.ptr)  # in place
    got = d_in.download((1, shape.D), np.float32)
    for l in range(1, N_LAYERS + 1):
        np.testing.assert_array_equal(ctx.read_topk(l, 1)[0], want_topk[l - 1], err_msg=f"layer {l} routing")
    # values grow by ~1e2 per layer; the bar is relative to the stack's own scale
    assert_close(got, want_x, "stack x_out", max_abs=1e-2 * N_LAYERS, rel_l2=1e-3)


def test_layered_kernels_match_stack_kernel(stack, monkeypatch):
    """The three-kernel path (used for T > 1) and the persistent kernel agree at T=1."""
    shape, layers, ctx = stack
    monkeypatch.setenv("GMOE_STACK_KERNEL", "0")
    ctx2 = gmoe.Context(shape, n_layers=2, max_tokens=1)
    try:
        ctx2.upload(1, layers[0])
        x = gmoe.activations(11, 4, 1, shape.D)
        a, sa = gmoe.forward_host(ctx, 1, x)
        b, sb = gmoe.forward_host(ctx2, 1, x)
    finally:
        ctx2.close()
    np.testing.assert_array_equal(sa["topk_idx"], sb["topk_idx"])
    assert np.array_equal(sa["xn"].view(np.uint32), sb["xn"].view(np.uint32))
    assert_close(a, b, "stack vs layered x_out", max_abs=1e-3, rel_l2=1e-5)


def test_forced_exact_router_matches_oracle(stack):
    """GMOE_FLAG_EXACT_ROUTER skips the certificate, so every layer takes the exact fp32
    replay of the router; routing and outputs must still match the oracle, and the
    one-launch stack must equal the certified run's routing."""
    shape, layers, ctx = stack
    x0 = gmoe.activations(11, 3, 1, shape.D)
    orc = oracle.Oracle("port")
    before = ctx.stats()["routing_exact_path"]
    x = x0.copy()
    for l in range(1, N_LAYERS + 1):
        print(f"[case] forced exact router, layer {l}", flush=True)
        want = orc.layer(shape, layers[l - 1], x)
        got, st = gmoe.forward_host(ctx, l, x, flags=gmoe.GMOE_FLAG_EXACT_ROUTER)
        np.testing.assert_array_equal(st["topk_idx"], want["topk_idx"], err_msg=f"layer {l} routing")
        # the replay is glm.c's fp32 chain with libm's expf bits
        assert np.array_equal(st["router_prob"].view(np.uint32), want["router_prob"].view(np.uint32)), f"layer {l} router_prob"
        assert np.array_equal(st["topk_w"].view(np.uint32), want["topk_w"].view(np.uint32)), f"layer {l} topk_w"
        assert_close(got, want["x_out"], f"layer {l} x_out")
        x = got
    assert ctx.stats()["routing_exact_path"] - before == N_LAYERS
    # the whole stack in one launch, forced exact, routes as the certified launch does
    d_in = gmoe.DeviceArray.from_numpy(x0)
    d_out = gmoe.DeviceArray(x0.nbytes)
    ctx.forward_layers(1, N_LAYERS, 1, d_in.ptr, d_out.ptr, flags=gmoe.GMOE_FLAG_EXACT_ROUTER)
    exact_topk = [ctx.read_topk(l, 1)[0] for l in range(1, N_LAYERS + 1)]
    ctx.forward_layers(1, N_LAYERS, 1, d_in.ptr, d_out.ptr)
    cert_topk = [ctx.read_topk(l, 1)[0] for l in range(1, N_LAYERS + 1)]
    for l in range(N_LAYERS):
        np.testing.assert_array_equal(exact_topk[l], cert_topk[l], err_msg=f"layer {l + 1}")
