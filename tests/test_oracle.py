"""The CPU restatement (oracle/moe_oracle.c) against glm.c's own code.

Two anchors: the committed fixtures in tests/golden/ (written by glm.c's infer.c,
built from the reference sources; see tests/golden/make_golden.py), and, where
oracle/_ref/libref_moe.so is built, a live bitwise comparison on fresh inputs.
Everything here is bit-exact: the restatement must reproduce glm.c's float
operations in glm.c's order.
"""
import numpy as np
import pytest

import gmoe
import oracle

from golden_data import GOLDEN, SMALL, load, with_ties_and_nan

OUT_KEYS = ["x_out", "xn", "router_prob", "topk_idx", "topk_w", "shared_out", "routed_out"]


def assert_bitwise(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    if got.dtype.kind == "f":
        same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    else:
        same = got == want
    bad = np.argwhere(~same)
    assert bad.size == 0, f"{what}: {len(bad)} elements differ, first at {tuple(bad[0])}: {got[tuple(bad[0])]!r} vs {want[tuple(bad[0])]!r}"


@pytest.fixture(scope="module")
def port():
    return oracle.Oracle("port")


def test_small_layer_matches_golden(port):
    g = load("small")
    hl = gmoe.HostLayer(SMALL, seed=7, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    res = port.layer(SMALL, hl, g["x"])
    for k in OUT_KEYS:
        assert_bitwise(res[k], g[k], k)


def test_small_layer_routed_off_matches_golden(port):
    g = load("small")
    hl = gmoe.HostLayer(SMALL, seed=7, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    res = port.layer(SMALL, hl, g["x"], disable_routed=True)
    assert_bitwise(res["x_out"], g["off_x_out"], "x_out with routed experts off")


def test_ties_and_nan_match_golden(port):
    """Exact ties in sel go to the lower expert index; a NaN probability is never chosen."""
    g = load("small")
    hl = with_ties_and_nan(gmoe.HostLayer(SMALL, seed=7, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM))
    res = port.layer(SMALL, hl, g["x"])
    for k in OUT_KEYS:
        assert_bitwise(res[k], g["tie_" + k], "tie " + k)
    assert (g["tie_topk_idx"][:, 0] == 3).all() and (g["tie_topk_idx"][:, 1] == 5).all()
    assert not (g["tie_topk_idx"] == 9).any()


def test_small_stack_matches_golden(port):
    g = load("small")
    layers = [gmoe.HostLayer(SMALL, seed=11, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM) for l in (1, 2, 3)]
    x, topk = port.stack(SMALL, layers, g["x"])
    assert_bitwise(x, g["stack_x_out"], "stack x_out")
    assert_bitwise(topk, g["stack_topk_idx"], "stack top-k")


def test_glm_layer_t1_matches_golden(port, glm_layer1):
    g = load("glm_t1")
    res = port.layer(gmoe.GLM47_FLASH, glm_layer1, g["x"])
    for k in OUT_KEYS:
        assert_bitwise(res[k], g[k], k)


def test_zipf_t128_matches_golden(port, glm_layer1_zipf):
    """Per-token top-k and the derived per-expert lists at T=128 with skewed routing."""
    g = load("dispatch_t128_zipf")
    x = gmoe.activations(0, 1, 128, gmoe.GLM47_FLASH.D)
    assert_bitwise(x[g["rows"]], g["x_rows"], "input rows")
    res = port.layer(gmoe.GLM47_FLASH, glm_layer1_zipf, x)
    assert_bitwise(res["topk_idx"], g["topk_idx"], "top-k")
    assert_bitwise(res["topk_w"], g["topk_w"], "top-k weights")
    assert_bitwise(res["x_out"][g["rows"]], g["x_out_rows"], "sampled output rows")
    offsets, tokens, slots = oracle.dispatch(res["topk_idx"], gmoe.GLM47_FLASH.E)
    assert_bitwise(offsets, g["offsets"], "expert offsets")
    assert_bitwise(tokens, g["tokens"], "expert token lists")
    assert_bitwise(slots, g["slots"], "expert slots")
    assert 0.3 < float(g["top4_share"]) < 0.5, "the Zipf workload should put ~40% of assignments on 4 experts"


@pytest.mark.skipif(not oracle.available("reference"), reason="oracle/_ref not built (needs the reference sources)")
class TestAgainstLiveReference:
    """Fresh inputs through both builds, compared bit for bit."""

    @pytest.fixture(scope="class")
    def ref(self):
        return oracle.Oracle("reference")

    @pytest.mark.parametrize("seed,norm_mode,T", [(1, gmoe.SYNTH_NORM_ONES, 1), (2, gmoe.SYNTH_NORM_RANDOM, 3),
                                                  (3, gmoe.SYNTH_NORM_RANDOM, 8)])
    def test_layer(self, port, ref, seed, norm_mode, T):
        hl = gmoe.HostLayer(SMALL, seed=seed, layer=2, norm_mode=norm_mode)
        x = gmoe.activations(seed, 5, T, SMALL.D) * np.float32(3.0)
        a, b = port.layer(SMALL, hl, x), ref.layer(SMALL, hl, x)
        for k in OUT_KEYS:
            assert_bitwise(a[k], b[k], k)

    def test_zipf_layer(self, port, ref):
        hl = gmoe.HostLayer(SMALL, seed=4, layer=1, bias_mode=gmoe.SYNTH_BIAS_ZIPF)
        x = gmoe.activations(4, 0, 16, SMALL.D)
        a, b = port.layer(SMALL, hl, x), ref.layer(SMALL, hl, x)
        for k in OUT_KEYS:
            assert_bitwise(a[k], b[k], k)

    def test_routed_off(self, port, ref):
        hl = gmoe.HostLayer(SMALL, seed=5, layer=1)
        x = gmoe.activations(5, 0, 2, SMALL.D)
        a = port.layer(SMALL, hl, x, disable_routed=True)
        b = ref.layer(SMALL, hl, x, disable_routed=True)
        for k in ("x_out", "shared_out", "routed_out", "topk_idx"):
            assert_bitwise(a[k], b[k], k)

    def test_stack(self, port, ref):
        layers = [gmoe.HostLayer(SMALL, seed=6, layer=l, norm_mode=gmoe.SYNTH_NORM_RANDOM) for l in (1, 2, 3, 4)]
        x = gmoe.activations(6, 0, 2, SMALL.D)
        xa, ta = port.stack(SMALL, layers, x)
        xb, tb = ref.stack(SMALL, layers, x)
        assert_bitwise(xa, xb, "stack x_out")
        assert_bitwise(ta, tb, "stack top-k")
