"""gmoe_forward_layers_noalloc: the decode entry point that allocates nothing, called through
the C ABI and compared with gmoe_forward_layers (same kernels, the context's workspace)
bit for bit, on two calls in a row, the second over fewer layers; and a run longer than
the fixed workspace holds is refused before anything is launched."""
import ctypes as C
import re

import numpy as np
import pytest

import gmoe
from conftest import DECODE_KERNELS, decode_kernel

pytestmark = pytest.mark.gpu

S = gmoe.GLM47_FLASH
N_UPLOADED = 5


@pytest.fixture(scope="module", params=list(DECODE_KERNELS))
def ctx(request):
    with decode_kernel(request.param):
        c = gmoe.Context(S, n_layers=21, max_tokens=1)
    for l in range(1, N_UPLOADED + 1):
        c.upload(l, gmoe.HostLayer(S, seed=31, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM))
    yield c
    c.close()


def noalloc(ctx, first, n, d_in, d_out):
    lib = ctx.lib
    lib.gmoe_forward_layers_noalloc.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int,
                                                C.c_void_p]
    lib.gmoe_forward_layers_noalloc.restype = C.c_int
    return lib.gmoe_forward_layers_noalloc(ctx.h, first, n, d_in.ptr, d_out.ptr, 0, None)


@pytest.mark.parametrize("first,n", [(1, 4), (2, 2)])
def test_noalloc_equals_forward_layers(ctx, first, n):
    x0 = gmoe.activations(31, first, 1, S.D)
    d_in = gmoe.DeviceArray.from_numpy(x0)
    d_out = gmoe.DeviceArray(x0.nbytes)
    print(f"[case] noalloc layers {first}..{first + n - 1}", flush=True)
    rc = noalloc(ctx, first, n, d_in, d_out)
    assert rc == 0, gmoe.last_error()
    got = d_out.download((1, S.D), np.float32)
    got_topk = [ctx.read_topk(l, 1)[0] for l in range(first, first + n)]
    print(f"[case] forward_layers layers {first}..{first + n - 1}", flush=True)
    ctx.forward_layers(first, n, 1, d_in.ptr, d_out.ptr)
    want = d_out.download((1, S.D), np.float32)
    want_topk = [ctx.read_topk(l, 1)[0] for l in range(first, first + n)]
    for l in range(n):
        np.testing.assert_array_equal(got_topk[l], want_topk[l], err_msg=f"layer {first + l} routing")
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "noalloc result differs from forward_layers"


def test_noalloc_refuses_a_run_longer_than_its_workspace(ctx):
    x0 = gmoe.activations(31, 9, 1, S.D)
    d_in = gmoe.DeviceArray.from_numpy(x0)
    d_out = gmoe.DeviceArray(x0.nbytes)
    print("[case] noalloc over 400 layers (more than the fixed array holds)", flush=True)
    rc = noalloc(ctx, 1, 400, d_in, d_out)
    assert rc == -1
    msg = gmoe.last_error()
    m = re.search(r"at most (\d+) layers", msg)
    assert m, msg
    assert N_UPLOADED <= int(m.group(1)) < 400, msg


def test_noalloc_at_group_size_16():
    """The exporter's form (group size 16, fp32 scales) on the same entry point: two calls in
    a row, the second over fewer layers, each equal to gmoe_forward_layers bit for bit."""
    s16 = gmoe.Shape(group_size=16)
    c = gmoe.Context(s16, n_layers=4, max_tokens=1)
    try:
        for l in range(1, 4):
            c.upload(l, gmoe.HostLayer(s16, seed=32, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                                       scale_mode=gmoe.SYNTH_SCALES_FP32))
        assert c.stats()["q8_form"] == gmoe.GMOE_Q8_TILED16
        for first, n in [(1, 3), (2, 1)]:
            x0 = gmoe.activations(32, first, 1, s16.D)
            d_in = gmoe.DeviceArray.from_numpy(x0)
            d_out = gmoe.DeviceArray(x0.nbytes)
            print(f"[case] noalloc gs=16 layers {first}..{first + n - 1}", flush=True)
            assert noalloc(c, first, n, d_in, d_out) == 0, gmoe.last_error()
            got = d_out.download((1, s16.D), np.float32)
            c.forward_layers(first, n, 1, d_in.ptr, d_out.ptr)
            want = d_out.download((1, s16.D), np.float32)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"gs=16 layers {first}+{n}"
    finally:
        c.close()
