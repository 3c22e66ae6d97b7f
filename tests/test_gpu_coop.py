"""The persistent decode kernels as cooperative launches (GMOE_COOPERATIVE=1, read when a
context is created): the runtime then guarantees that the whole grid is resident at once,
which the kernels' cross-block waits need, instead of relying on an otherwise idle GPU.
The results must equal the ordinary launch's bit for bit, routing included, on every
persistent kernel, and a captured graph (which takes the ordinary form) must still replay."""
import os

import numpy as np
import pytest

import gmoe
from conftest import decode_kernel, launched, assert_decode_kernel

pytestmark = pytest.mark.gpu

S = gmoe.GLM47_FLASH
N = 6


def run(kind, coop, layers):
    old = os.environ.get("GMOE_COOPERATIVE")
    os.environ["GMOE_COOPERATIVE"] = "1" if coop else "0"
    try:
        with decode_kernel(kind):
            ctx = gmoe.Context(S, n_layers=N + 1, max_tokens=1)
    finally:
        if old is None:
            os.environ.pop("GMOE_COOPERATIVE", None)
        else:
            os.environ["GMOE_COOPERATIVE"] = old
    try:
        for l, hl in enumerate(layers, start=1):
            ctx.upload(l, hl)
        x = gmoe.activations(43, 0, 1, S.D)
        d_in = gmoe.DeviceArray.from_numpy(x)
        d_out = gmoe.DeviceArray(x.nbytes)
        outs = []

        def step():
            ctx.forward_layers(1, N, 1, d_in.ptr, d_out.ptr)

        ran = launched(ctx, step)
        assert_decode_kernel(ran, kind)
        for _ in range(3):
            step()
            outs.append(d_out.download((1, S.D), np.float32))
        topk = [ctx.read_topk(l, 1)[0] for l in range(1, N + 1)]
        assert ctx.stats()["tokens_routed"] > 0
        return outs, topk
    finally:
        ctx.close()


@pytest.fixture(scope="module")
def layers():
    return [gmoe.HostLayer(S, seed=43, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM) for l in range(1, N + 1)]


@pytest.mark.parametrize("kind", ["relay", "stack"])
def test_cooperative_launch_equals_the_ordinary_one(layers, kind):
    print(f"[case] cooperative {kind}", flush=True)
    want, want_topk = run(kind, False, layers)
    got, got_topk = run(kind, True, layers)
    for l in range(N):
        np.testing.assert_array_equal(got_topk[l], want_topk[l], err_msg=f"layer {l + 1} routing")
    for w, g in zip(want, got):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))
