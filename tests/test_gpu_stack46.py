"""The benchmark's workload at full depth: 46 GLM-4.7-Flash MoE layers (seed 0, as bench.py
uploads them), one token through one persistent launch.

* The one launch equals 46 single-layer launches bit for bit (every layer's workspace,
  counters and flags of the launch are exercised, not just the first few).
* Every layer's routing equals the oracle's on that layer's own GPU input, with xn bit
  for bit and the layer's outputs within the bar.
* The final x is within the bar of the oracle's 46-layer stack (the decode loop of
  infer.c:1818-1860, MoE half), the max-abs bar summed over the layers."""
import numpy as np
import pytest

import gmoe
import oracle
from conftest import DECODE_KERNEL_NAMES, assert_close, assert_decode_kernel, decode_kernel, launched

pytestmark = pytest.mark.gpu

N_LAYERS = 46


@pytest.fixture(scope="module", params=list(DECODE_KERNEL_NAMES))
def stack46(request):
    shape = gmoe.GLM47_FLASH
    with decode_kernel(request.param):
        ctx = gmoe.Context(shape, n_layers=N_LAYERS + 1, max_tokens=1)
    ctx.kind = request.param
    layers = []
    for l in range(1, N_LAYERS + 1):
        hl = gmoe.HostLayer(shape, seed=0, layer=l)
        ctx.upload(l, hl)
        layers.append(hl)
        if l % 10 == 0:
            print(f"[setup] uploaded {l} of {N_LAYERS} layers", flush=True)
    yield shape, layers, ctx
    ctx.close()


def test_46_layers_one_launch_against_oracle(stack46):
    shape, layers, ctx = stack46
    x0 = gmoe.activations(0, 0, 1, shape.D)  # the benchmark's input
    print(f"[case] 46 layers in one persistent launch ({ctx.kind})", flush=True)
    d_in = gmoe.DeviceArray.from_numpy(x0)
    d_out = gmoe.DeviceArray(x0.nbytes)
    ran = launched(ctx, lambda: ctx.forward_layers(1, N_LAYERS, 1, d_in.ptr, d_out.ptr))
    assert_decode_kernel(ran, ctx.kind)
    x_one = d_out.download((1, shape.D), np.float32)
    topk_one = [ctx.read_topk(l, 1)[0] for l in range(1, N_LAYERS + 1)]

    orc = oracle.Oracle("port")
    x = x0.copy()
    for l in range(1, N_LAYERS + 1):
        want = orc.layer(shape, layers[l - 1], x)
        got, st = gmoe.forward_host(ctx, l, x)
        np.testing.assert_array_equal(st["topk_idx"], want["topk_idx"], err_msg=f"layer {l} routing vs oracle")
        np.testing.assert_array_equal(topk_one[l - 1], st["topk_idx"], err_msg=f"layer {l}: one launch vs per layer")
        assert np.array_equal(st["xn"].view(np.uint32), want["xn"].view(np.uint32)), f"layer {l} xn"
        assert_close(st["topk_w"], want["topk_w"], f"layer {l} topk_w", max_abs=1e-5, rel_l2=1e-5)
        assert_close(st["shared_out"], want["shared_out"], f"layer {l} shared_out")
        assert_close(st["routed_out"], want["routed_out"], f"layer {l} routed_out")
        assert_close(got, want["x_out"], f"layer {l} x_out")
        x = got
        if l % 10 == 0:
            print(f"[case] layers 1..{l} match the oracle", flush=True)
    assert np.array_equal(x.view(np.uint32), x_one.view(np.uint32)), "one launch differs from 46 single-layer launches"

    want_x, want_topk = orc.stack(shape, layers, x0)
    for l in range(N_LAYERS):
        np.testing.assert_array_equal(topk_one[l], want_topk[l], err_msg=f"layer {l + 1} vs the oracle's stack")
    # each layer's own error is within the bar; over the stack they add up (as in the 6-layer test)
    assert_close(x_one, want_x, "46-layer x", max_abs=1e-2 * N_LAYERS, rel_l2=1e-3)
