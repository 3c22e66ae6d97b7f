"""The residual of a decode launch, on both T=1 kernels, against the launch's own observables.

glm.c's residual is x' = fl(x + fl(shared + acc)) (infer.c:1192, 1212-1214). k_moe_stack
stores exactly that. k_moe_relay hands x on between layers as words that carry the layer's
parity in their lowest bit, so its x (the launch's output too, so that one launch of n
layers equals n launches of one) is that value rounded to an even significand: an odd
significand goes to the even neighbour whose bit 1 is clear, up or down, so the rounding
has no direction on average. Clearing the lowest bit instead (toward zero every time)
fails here on the rows whose bit 1 is set. Both rules are checked bit for bit on every row
of a one-layer launch, with the rows that round up and down counted."""
import numpy as np
import pytest

import gmoe
from conftest import assert_decode_kernel, launched

pytestmark = pytest.mark.gpu

SHAPE = gmoe.Shape(dim=2048, moe_ffn_dim=1536, n_routed_experts=64, n_experts_used=4)


def round_even_bit1(v):
    """v (float32) with an odd significand moved to the even neighbour whose bit 1 is clear."""
    b = v.view(np.uint32).copy()
    odd = (b & 1) == 1
    up = odd & ((b & 2) == 2)
    b[up] += 1
    b[odd & ~up] -= 1
    return b.view(np.float32)


@pytest.mark.parametrize("seed", [3, 11])
def test_one_layer_launch_residual(dkernel, seed):
    ctx = gmoe.Context(SHAPE, n_layers=2, max_tokens=1)
    try:
        ctx.upload(1, gmoe.HostLayer(SHAPE, seed=seed, layer=1))
        rng = np.random.default_rng(seed)
        x = rng.standard_normal((1, SHAPE.D)).astype(np.float32)
        print(f"[case] {dkernel} seed {seed}: one-layer launch", flush=True)
        out = {}

        def run():
            out["x"], out["st"] = gmoe.forward_host(ctx, 1, x)

        assert_decode_kernel(launched(ctx, run), dkernel)
        st = out["st"]
        exact = x[0] + (st["shared_out"][0] + st["routed_out"][0])
        assert exact.dtype == np.float32
        bits = exact.view(np.uint32)
        n_up = int(np.count_nonzero((bits & 3) == 3))
        n_down = int(np.count_nonzero((bits & 3) == 1))
        assert n_up > SHAPE.D // 8 and n_down > SHAPE.D // 8, "the check needs rows that round each way"
        want = round_even_bit1(exact) if dkernel == "relay" else exact
        got = out["x"][0]
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, f"{bad.size} rows differ from the {dkernel} kernel's residual rule, first at {bad[:4]}"
    finally:
        ctx.close()
