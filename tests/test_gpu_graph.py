"""A persistent decode launch captured in a HIP graph and replayed.

k_moe_relay hands its phases' results over as words tagged with a per-layer parity that the
launch's reset kernel flips in device memory, so a replayed launch must flip it again
rather than reuse the parity of the capture. The graph is replayed several times on inputs
that change between replays, with eager launches of the same context interleaved, and
every replay must equal the eager result for its input bit for bit (routing included).
The no-alloc entry point is captured the same way: it clears its fixed workspace with a
kernel, which a replay repeats."""
import ctypes as C

import numpy as np
import pytest

import gmoe
from conftest import decode_kernel

pytestmark = pytest.mark.gpu

S = gmoe.GLM47_FLASH
N = 4


@pytest.fixture(scope="module")
def relay_ctx():
    with decode_kernel("relay"):
        ctx = gmoe.Context(S, n_layers=N + 1, max_tokens=1)
    for l in range(1, N + 1):
        ctx.upload(l, gmoe.HostLayer(S, seed=41, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM))
    yield ctx
    ctx.close()


def capture(stream, call):
    hip = gmoe.hip()
    gmoe.hip_check(hip.hipStreamBeginCapture(stream.h, 0), "hipStreamBeginCapture")
    call()
    graph = C.c_void_p()
    gmoe.hip_check(hip.hipStreamEndCapture(stream.h, C.byref(graph)), "hipStreamEndCapture")
    exe = C.c_void_p()
    gmoe.hip_check(hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
    return graph, exe


def eager(ctx, x):
    d_in = gmoe.DeviceArray.from_numpy(x)
    d_out = gmoe.DeviceArray(x.nbytes)
    ctx.forward_layers(1, N, 1, d_in.ptr, d_out.ptr)
    out = d_out.download((1, S.D), np.float32)
    topk = [ctx.read_topk(l, 1)[0] for l in range(1, N + 1)]
    return out, topk


@pytest.mark.parametrize("entry", ["forward_layers", "noalloc"])
def test_replays_equal_eager_launches(relay_ctx, entry):
    ctx = relay_ctx
    hip = gmoe.hip()
    xs = [gmoe.activations(41, 10 + i, 1, S.D) for i in range(3)]
    want = [eager(ctx, x) for x in xs]
    d_in = gmoe.DeviceArray(xs[0].nbytes)
    d_out = gmoe.DeviceArray(xs[0].nbytes)
    stream = gmoe.Stream()
    lib = ctx.lib
    lib.gmoe_forward_layers_noalloc.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int,
                                                C.c_void_p]
    lib.gmoe_forward_layers_noalloc.restype = C.c_int

    def call():
        if entry == "noalloc":
            rc = lib.gmoe_forward_layers_noalloc(ctx.h, 1, N, d_in.ptr, d_out.ptr, 0, stream.h)
            assert rc == 0, gmoe.last_error()
        else:
            ctx.forward_layers(1, N, 1, d_in.ptr, d_out.ptr, stream=stream.h)

    print(f"[case] {entry}: capture of a {N}-layer relay launch", flush=True)
    graph, exe = capture(stream, call)
    try:
        for rep, i in enumerate([0, 1, 2, 0, 2, 1]):
            print(f"[case] {entry}: replay {rep} on input {i}", flush=True)
            d_in.upload(xs[i])
            gmoe.hip_check(hip.hipGraphLaunch(exe, stream.h), "hipGraphLaunch")
            stream.sync()
            got = d_out.download((1, S.D), np.float32)
            topk = [ctx.read_topk(l, 1)[0] for l in range(1, N + 1)]
            for l in range(N):
                np.testing.assert_array_equal(topk[l], want[i][1][l], err_msg=f"replay {rep} layer {l + 1} routing")
            assert np.array_equal(got.view(np.uint32), want[i][0].view(np.uint32)), f"replay {rep} differs"
            # eager work of the same context between the replays
            out, _ = eager(ctx, xs[(i + 1) % 3])
            assert np.array_equal(out.view(np.uint32), want[(i + 1) % 3][0].view(np.uint32)), "eager launch differs"
    finally:
        hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
