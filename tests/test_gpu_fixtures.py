"""The small golden fixture (tests/golden/small.npz, written by glm.c's own infer.c) on the GPU:
the base layer, the variant with an exact router tie and a NaN router row, the routed
experts switched off, and a 3-layer stack. Each token is also run on its own, as glm.c's
decode does (infer.c:2190-2233), so the persistent decode kernel sees every case too.

Bar: top-k indices exact (ties to the lower expert index, NaN never chosen,
infer.c:1110-1135); xn bit-identical; router probabilities and normalised weights within
1e-5 (NaN where glm.c has NaN); float outputs within max-abs 1e-2 and rel-L2 1e-3."""
import numpy as np
import pytest

import gmoe
from conftest import assert_close
from golden_data import SMALL, load, with_ties_and_nan

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def golden():
    return load("small")


def base_layer():
    return gmoe.HostLayer(SMALL, seed=7, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM)


def assert_prob_close(got, want, what):
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), f"{what}: NaN pattern differs"
    assert_close(got[~nan], want[~nan], what, max_abs=1e-5, rel_l2=1e-5)


def check_layer(st, got, g, prefix, what):
    np.testing.assert_array_equal(st["topk_idx"], g[prefix + "topk_idx"], err_msg=f"{what}: top-k indices")
    assert np.array_equal(st["xn"].view(np.uint32), g[prefix + "xn"].view(np.uint32)), f"{what}: xn bits"
    assert_prob_close(st["router_prob"], g[prefix + "router_prob"], f"{what}: router_prob")
    assert_close(st["topk_w"], g[prefix + "topk_w"], f"{what}: topk_w", max_abs=1e-5, rel_l2=1e-5)
    assert_close(st["shared_out"], g[prefix + "shared_out"], f"{what}: shared_out")
    assert_close(st["routed_out"], g[prefix + "routed_out"], f"{what}: routed_out")
    assert_close(got, g[prefix + "x_out"], f"{what}: x_out")


@pytest.mark.parametrize("variant", ["base", "tie_nan"])
@pytest.mark.parametrize("per_token", [False, True])
def test_layer_against_fixture(golden, dkernel, variant, per_token):
    g = golden
    hl = base_layer()
    if variant == "tie_nan":
        hl = with_ties_and_nan(hl)
    prefix = "" if variant == "base" else "tie_"
    ctx = gmoe.Context(SMALL, n_layers=2, max_tokens=4)
    try:
        ctx.upload(1, hl)
        if per_token:
            for t in range(g["x"].shape[0]):
                print(f"[case] small.npz {variant} token {t} (T=1, persistent kernel)", flush=True)
                got, st = gmoe.forward_host(ctx, 1, g["x"][t:t + 1])
                one = {k: g[prefix + k][t:t + 1] for k in ("topk_idx", "xn", "router_prob", "topk_w", "shared_out",
                                                           "routed_out", "x_out")}
                check_layer(st, got, {prefix + k: v for k, v in one.items()}, prefix, f"{variant} token {t}")
        else:
            print(f"[case] small.npz {variant} T=4 batch", flush=True)
            got, st = gmoe.forward_host(ctx, 1, g["x"])
            check_layer(st, got, g, prefix, f"{variant} T=4")
    finally:
        ctx.close()


def test_tie_goes_to_the_lower_index_and_nan_is_never_chosen(golden, dkernel):
    """The fixture's own facts, restated on the GPU's routing: experts 3 and 5 tie exactly
    and 3 ranks first, expert 9 (NaN) is never selected."""
    hl = with_ties_and_nan(base_layer())
    ctx = gmoe.Context(SMALL, n_layers=2, max_tokens=4)
    try:
        ctx.upload(1, hl)
        print("[case] small.npz tie/NaN facts", flush=True)
        _, st = gmoe.forward_host(ctx, 1, golden["x"])
        stats = ctx.stats()
    finally:
        ctx.close()
    idx = st["topk_idx"]
    assert np.all(idx[:, 0] == 3) and np.all(idx[:, 1] == 5)
    assert not np.any(idx == 9)
    assert stats["routing_exact_path"] >= 4  # an exact tie is never certified: the replay decides it


def test_routed_off_against_fixture(golden, dkernel):
    ctx = gmoe.Context(SMALL, n_layers=2, max_tokens=4)
    try:
        ctx.upload(1, base_layer())
        print("[case] small.npz routed experts off, T=4", flush=True)
        got, st = gmoe.forward_host(ctx, 1, golden["x"], flags=gmoe.GMOE_FLAG_NO_ROUTED)
        assert_close(got, golden["off_x_out"], "off x_out")
        assert np.all(st["routed_out"] == 0)
        for t in range(golden["x"].shape[0]):
            print(f"[case] small.npz routed experts off, token {t}", flush=True)
            got1, _ = gmoe.forward_host(ctx, 1, golden["x"][t:t + 1], flags=gmoe.GMOE_FLAG_NO_ROUTED)
            assert_close(got1, golden["off_x_out"][t:t + 1], f"off x_out token {t}")
    finally:
        ctx.close()


def test_three_layer_stack_against_fixture(golden, dkernel):
    """Layers 1-3 (seed 11): the batch through gmoe_forward_layers (grouped path per layer)
    and each token through one persistent launch over the three layers."""
    layers = [gmoe.HostLayer(SMALL, seed=11, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM) for l in (1, 2, 3)]
    ctx = gmoe.Context(SMALL, n_layers=4, max_tokens=4)
    try:
        for l, hl in enumerate(layers, start=1):
            ctx.upload(l, hl)
        x = golden["x"]
        print("[case] small.npz 3-layer stack, T=4", flush=True)
        d = gmoe.DeviceArray.from_numpy(x)
        ctx.forward_layers(1, 3, 4, d.ptr, d.ptr)
        got = d.download(x.shape, np.float32)
        for l in range(3):
            np.testing.assert_array_equal(ctx.read_topk(l + 1, 4)[0], golden["stack_topk_idx"][l],
                                          err_msg=f"batch layer {l + 1} top-k")
        assert_close(got, golden["stack_x_out"], "stack x_out (T=4)", max_abs=3e-2)
        for t in range(x.shape[0]):
            print(f"[case] small.npz 3-layer stack, token {t} (one persistent launch)", flush=True)
            d1 = gmoe.DeviceArray.from_numpy(x[t:t + 1])
            ctx.forward_layers(1, 3, 1, d1.ptr, d1.ptr)
            got1 = d1.download((1, SMALL.D), np.float32)
            for l in range(3):
                np.testing.assert_array_equal(ctx.read_topk(l + 1, 1)[0][0], golden["stack_topk_idx"][l][t],
                                              err_msg=f"token {t} layer {l + 1} top-k")
            assert_close(got1, golden["stack_x_out"][t:t + 1], f"stack x_out token {t}", max_abs=3e-2)
    finally:
        ctx.close()

