"""The routers' certificates under heavy cancellation.

glm.c's logit is a sequential fp32 chain (infer.c:916-938); the decode kernel and
the batch routers estimate it in fp64 and certify the top-k only when the chain's
rounding bound separates the candidates, else they replay the chain exactly. These cases build two
router rows whose products climb to partial sums near D/2 and return near zero, so
that the chains' roundings (ulps of ~1e3) exceed the rows' exact difference (3e-4 to
6e-4), which is chosen so that the fp32 chain orders the pair against the exact order.
Biases make the pair compete for the last top-k slot. A bound below that difference
would certify the exact order and pick the wrong expert; the routing must equal the
oracle's, for a layer run on its own and for the second layer of a one-launch stack
(whose input is the first layer's output, held on the GPU)."""
import math

import numpy as np
import pytest

import gmoe
import oracle
from conftest import assert_close

SHAPE = gmoe.Shape(dim=2048, moe_ffn_dim=256, n_routed_experts=64, n_experts_used=4)
PAIR = (10, 11)


def chain32(g, xn):
    """glm.c's logit: fp32 products, summed in order in fp32."""
    p = np.multiply(g, xn, dtype=np.float32)
    return float(np.add.accumulate(p, dtype=np.float32)[-1])


def exact(g, xn):
    return math.fsum((g.astype(np.float64) * xn.astype(np.float64)).tolist())


def adversarial_rows(xn, rng):
    """Two rows whose fp32 chains order them against their exact logits, with exact
    logits 3e-4 to 6e-4 apart: a certificate whose bound fell below that would certify
    the exact order. The chain is monotone in each product, so the second row moves
    products both ways: +d at 400 columns where the partial sums are near D/2 (d below
    half their ulp, so each step rounds it away or up to an ulp at random: noise ~6e-4)
    and minus their total less eps near the end, where the partial sums are small and
    keep it; the exact difference is +eps."""
    D = xn.size
    m = rng.uniform(0.5, 1.5, D)
    p = np.where(np.arange(D) < D // 2, m, -m)
    p[-1] += 0.3 - p.sum()  # the exact sum near 0.3: sigmoid away from saturation
    nz = xn != 0
    safe = np.where(nz, xn, 1.0).astype(np.float64)
    g1 = np.where(nz, p / safe, 0.0).astype(np.float32)
    c1, e1 = chain32(g1, xn), exact(g1, xn)
    for _ in range(1000):
        ks = rng.choice(np.arange(D // 2 - 500, D // 2 + 500), 400, replace=False)
        ks = ks[nz[ks]]
        k2 = int(rng.integers(D - 8, D - 1))
        if not nz[k2]:
            continue
        d = rng.uniform(1e-5, 3e-5, ks.size)
        eps = rng.uniform(3e-4, 6e-4)
        g2 = g1.copy()
        g2[ks] = ((g1[ks].astype(np.float64) * xn[ks] + d) / xn[ks]).astype(np.float32)
        # the exact change of the moved products, so that the end compensates it to eps
        moved = math.fsum(((g2[ks].astype(np.float64) - g1[ks]) * xn[ks]).tolist())
        g2[k2] = np.float32((float(g1[k2]) * float(xn[k2]) - (moved - eps)) / float(xn[k2]))
        c2, e2 = chain32(g2, xn), exact(g2, xn)
        # the chains apart by 5e-5 or more, so that the scores' order never hinges on
        # expf's last bits
        if (c1 < c2) != (e1 < e2) and abs(c1 - c2) > 5e-5 and abs(e1 - e2) > 2.5e-4:
            return g1, g2
    raise AssertionError("no order-flipping pair found")


def make_adversarial(L, xn, rng, shape=SHAPE):
    g1, g2 = adversarial_rows(xn, rng)
    L.gate_inp[PAIR[0]] = g1
    L.gate_inp[PAIR[1]] = g2
    b = np.full(shape.E, -10.0, np.float32)
    b[:shape.K - 1] = 10.0 * np.arange(shape.K - 1, 0, -1)  # certainly selected, in order, never tied
    b[list(PAIR)] = 0.0  # the pair competes for the last slot
    L.exp_probs_b[:] = b


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [21, 22, 23])
def test_cancellation_routing_against_oracle(seed):
    rng = np.random.default_rng(seed)
    orc = oracle.Oracle("port")
    L1 = gmoe.HostLayer(SHAPE, seed=seed, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    L2 = gmoe.HostLayer(SHAPE, seed=seed, layer=2, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    x = gmoe.activations(seed, 7, 1, SHAPE.D)
    make_adversarial(L1, orc.layer(SHAPE, L1, x)["xn"][0], rng)
    ctx = gmoe.Context(SHAPE, n_layers=3, max_tokens=1)
    try:
        ctx.upload(1, L1)
        print(f"[case] cancellation seed={seed} layer 1", flush=True)
        want1 = orc.layer(SHAPE, L1, x)
        got1, st1 = gmoe.forward_host(ctx, 1, x)
        np.testing.assert_array_equal(st1["topk_idx"], want1["topk_idx"], err_msg="layer 1 routing")
        assert_close(got1, want1["x_out"], "layer 1 x_out")
        # layer 2's rows against the xn of the GPU's own layer-1 output
        make_adversarial(L2, orc.layer(SHAPE, L2, got1)["xn"][0], rng)
        ctx.upload(2, L2)
        print(f"[case] cancellation seed={seed} layers 1-2 in one launch", flush=True)
        want2 = orc.layer(SHAPE, L2, got1)
        d_in = gmoe.DeviceArray.from_numpy(x)
        d_out = gmoe.DeviceArray(x.nbytes)
        ctx.forward_layers(1, 2, 1, d_in.ptr, d_out.ptr)
        np.testing.assert_array_equal(ctx.read_topk(1, 1)[0], want1["topk_idx"], err_msg="stack layer 1 routing")
        np.testing.assert_array_equal(ctx.read_topk(2, 1)[0], want2["topk_idx"], err_msg="stack layer 2 routing")
        assert_close(d_out.download((1, SHAPE.D), np.float32), want2["x_out"], "stack x_out")
    finally:
        ctx.close()


@pytest.mark.gpu
@pytest.mark.parametrize("E", [64, 128])
def test_cancellation_routing_relay(E):
    """The cancellation at T=1 on k_moe_relay (moe_ffn_dim 512: enough expert items for its
    combine chunks): no certificate holds, and the replay runs on the few experts that can
    still be chosen (the K - 1 certainly selected ones and the pair)."""
    shape = gmoe.Shape(dim=2048, moe_ffn_dim=512, n_routed_experts=E, n_experts_used=4)
    rng = np.random.default_rng(41 + E)
    orc = oracle.Oracle("port")
    L = gmoe.HostLayer(shape, seed=41, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    x = gmoe.activations(41, 7, 1, shape.D)
    make_adversarial(L, orc.layer(shape, L, x)["xn"][0], rng, shape)
    ctx = gmoe.Context(shape, n_layers=2, max_tokens=1)
    try:
        ctx.upload(1, L)
        ctx.profile(True)
        print(f"[case] cancellation on k_moe_relay E={E}", flush=True)
        want = orc.layer(shape, L, x)
        got, st = gmoe.forward_host(ctx, 1, x)
        np.testing.assert_array_equal(st["topk_idx"], want["topk_idx"], err_msg="relay routing")
        assert_close(got, want["x_out"], "relay x_out")
        assert "k_moe_relay" in ctx.profile_read()
        stats = ctx.stats()
        assert stats["routing_exact_path"] >= 1 and stats["routing_exact_subset"] >= 1, stats
    finally:
        ctx.close()


@pytest.mark.gpu
@pytest.mark.parametrize("E", [64, 128])
def test_cancellation_routing_batch(E):
    """The batch router's certificates under the same cancellation: with 64 experts the
    four-quarter partial sums and their joined bound, with 128 the one-block-per-token
    router. Other tokens would meet the rows' large norms and tie at a saturated sigmoid,
    so the batch repeats the adversarial token."""
    shape = gmoe.Shape(dim=2048, moe_ffn_dim=256, n_routed_experts=E, n_experts_used=4)
    T = 8
    rng = np.random.default_rng(31 + E)
    orc = oracle.Oracle("port")
    L = gmoe.HostLayer(shape, seed=31, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    x = np.repeat(gmoe.activations(31, 7, 1, shape.D), T, axis=0)
    make_adversarial(L, orc.layer(shape, L, x[:1])["xn"][0], rng, shape)
    ctx = gmoe.Context(shape, n_layers=2, max_tokens=T)
    try:
        ctx.upload(1, L)
        print(f"[case] cancellation batch E={E} T={T}", flush=True)
        want = orc.layer(shape, L, x)
        got, st = gmoe.forward_host(ctx, 1, x)
        np.testing.assert_array_equal(st["topk_idx"], want["topk_idx"], err_msg="batch routing")
        assert_close(got, want["x_out"], "batch x_out")
        stats = ctx.stats()
        assert stats["routing_exact_path"] >= T  # no certificate may hold at this cancellation
        # only the K - 1 certainly selected experts and the pair can still be chosen: the
        # replay runs on those five, not on every expert
        assert stats["routing_exact_subset"] >= T
    finally:
        ctx.close()


@pytest.mark.gpu
@pytest.mark.parametrize("E,T", [(64, 8), (128, 8), (64, 1), (128, 1)])
def test_all_experts_tied_batch(E, T):
    """Every expert's gate row the same and no bias: all E scores tie exactly, so no
    certificate holds and no expert can be ruled out. The router (the batch routers at
    T=8, the decode kernel at T=1) then replays every expert's chain (more than the subset
    replay holds), and glm.c's insertion top-k breaks the tie by index: experts 0..K-1, in
    that order."""
    # at T=1, moe_ffn_dim 512 so that the shape runs on k_moe_relay
    shape = gmoe.Shape(dim=2048, moe_ffn_dim=512 if T == 1 else 256, n_routed_experts=E, n_experts_used=4)
    orc = oracle.Oracle("port")
    L = gmoe.HostLayer(shape, seed=41, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    L.gate_inp[:] = L.gate_inp[0]
    L.exp_probs_b[:] = 0.0
    x = gmoe.activations(41, 7, T, shape.D)
    ctx = gmoe.Context(shape, n_layers=2, max_tokens=T)
    try:
        ctx.upload(1, L)
        print(f"[case] all experts tied E={E} T={T}", flush=True)
        want = orc.layer(shape, L, x)
        got, st = gmoe.forward_host(ctx, 1, x)
        np.testing.assert_array_equal(st["topk_idx"], want["topk_idx"], err_msg="tied routing")
        assert np.all(st["topk_idx"] == np.arange(shape.K))
        assert_close(got, want["x_out"], "tied x_out")
        stats = ctx.stats()
        assert stats["routing_exact_path"] >= T
        assert stats["routing_exact_subset"] == 0
    finally:
        ctx.close()


def test_adversarial_rows_flip_the_order():
    """The construction itself (CPU): the chains order the pair against exact sums
    3e-4 to 6e-4 apart."""
    rng = np.random.default_rng(5)
    xn = rng.standard_normal(SHAPE.D).astype(np.float32)
    g1, g2 = adversarial_rows(xn, rng)
    c1, c2, e1, e2 = chain32(g1, xn), chain32(g2, xn), exact(g1, xn), exact(g2, xn)
    assert (c1 < c2) != (e1 < e2) and abs(c1 - c2) > 5e-5
    assert 2.5e-4 < abs(e1 - e2) < 7e-4 and abs(e1 - 0.3) < 0.1

