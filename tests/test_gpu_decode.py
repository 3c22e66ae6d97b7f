"""Decode (T=1 and small T) parity of the HIP MoE layer against the oracle.

Each token of a batch is an independent decode step (infer.c:2190-2233), so a
batch of T tokens checks T decode cases at once; T=1 is checked on its own too.
Bar: top-k indices exact, xn bitwise (both pinned to glm.c's arithmetic), float
outputs within max-abs 1e-2 and rel-L2 1e-3."""
import os

import numpy as np
import pytest

import gmoe
import oracle
from conftest import DECODE_KERNELS, assert_close, assert_decode_kernel, current_decode_kernel, decode_kernel, launched

pytestmark = pytest.mark.gpu

SMALL = gmoe.Shape(dim=256, moe_ffn_dim=256, n_routed_experts=16, n_experts_used=4)
# more experts than a wave's lanes: decode router blocks hold several experts each, the
# batch router takes its one-block-per-token form (k_router_tok), selection spans chunks
WIDE = gmoe.Shape(dim=512, moe_ffn_dim=256, n_routed_experts=128, n_experts_used=6)
WIDEST = gmoe.Shape(dim=256, moe_ffn_dim=256, n_routed_experts=256, n_experts_used=8)


def run_case(shape, seed, T, norm_mode=gmoe.SYNTH_NORM_ONES, flags=0, layer=1, expect=None):
    print(f"[case] D={shape.D} F={shape.F} E={shape.E} K={shape.K} seed={seed} T={T} norm={norm_mode} flags={flags}",
          flush=True)
    L = gmoe.HostLayer(shape, seed=seed, layer=layer, norm_mode=norm_mode)
    x = gmoe.activations(seed, 100 + layer, T, shape.D)
    want = oracle.Oracle("port").layer(shape, L, x, disable_routed=bool(flags & gmoe.GMOE_FLAG_NO_ROUTED))
    ctx = gmoe.Context(shape, n_layers=layer + 1, max_tokens=T)
    try:
        ctx.upload(layer, L)
        out = {}
        ran = launched(ctx, lambda: out.update(r=gmoe.forward_host(ctx, layer, x, flags=flags)))
        got, st = out["r"]
        if expect is not None:  # the kernels the case must have run
            assert expect <= ran, ran
        elif T == 1:  # the persistent kernel the environment asks for
            assert_decode_kernel(ran, current_decode_kernel())
        stats = ctx.stats()
    finally:
        ctx.close()
    return want, got, st, stats


def check(want, got, st, stats):
    np.testing.assert_array_equal(st["topk_idx"], want["topk_idx"], err_msg="top-k indices")
    assert np.array_equal(st["xn"].view(np.uint32), want["xn"].view(np.uint32)), "xn not bit-identical"
    assert_close(st["router_prob"], want["router_prob"], "router_prob", max_abs=1e-5, rel_l2=1e-5)
    assert_close(st["topk_w"], want["topk_w"], "topk_w", max_abs=1e-5, rel_l2=1e-5)
    assert_close(st["shared_out"], want["shared_out"], "shared_out")
    assert_close(st["routed_out"], want["routed_out"], "routed_out")
    assert_close(got, want["x_out"], "x_out")


def test_small_t1(dkernel):
    check(*run_case(SMALL, seed=1, T=1))


def test_small_batch_random_norm():
    check(*run_case(SMALL, seed=2, T=16, norm_mode=gmoe.SYNTH_NORM_RANDOM))


def test_small_no_routed():
    want, got, st, stats = run_case(SMALL, seed=3, T=4, flags=gmoe.GMOE_FLAG_NO_ROUTED)
    check(want, got, st, stats)
    assert np.all(st["routed_out"] == 0)


def test_glm_shape_t1(dkernel):
    check(*run_case(gmoe.GLM47_FLASH, seed=0, T=1))


def test_glm_shape_batch8():
    check(*run_case(gmoe.GLM47_FLASH, seed=5, T=8, norm_mode=gmoe.SYNTH_NORM_RANDOM))


@pytest.mark.parametrize("T", [1, 8])
def test_per_token_kernels_against_oracle(monkeypatch, T):
    """The per-token kernels (the router, k_gate_up, k_down_combine) on their own: with the
    persistent kernels off (GMOE_STACK_KERNEL=0) a T=1 call takes them, and with
    GMOE_GROUPED_MIN_T above T so does a batch."""
    monkeypatch.setenv("GMOE_STACK_KERNEL", "0")
    monkeypatch.setenv("GMOE_GROUPED_MIN_T", "64")
    want, got, st, stats = run_case(gmoe.GLM47_FLASH, seed=6, T=T, norm_mode=gmoe.SYNTH_NORM_RANDOM,
                                    expect={"gate_up", "down"})
    check(want, got, st, stats)


@pytest.mark.parametrize("T,kind", [(1, "stack"), (1, "relay"), (8, "stack")])
def test_wide_expert_count(T, kind):
    with decode_kernel(kind):
        check(*run_case(WIDE, seed=6, T=T, norm_mode=gmoe.SYNTH_NORM_RANDOM))


@pytest.mark.parametrize("T,kind", [(1, "stack"), (1, "relay"), (8, "stack")])
def test_widest_expert_count(T, kind):
    with decode_kernel(kind):
        check(*run_case(WIDEST, seed=7, T=T))


@pytest.mark.parametrize("name,T", [("small", 16), ("glm", 8), ("wide", 8)])
def test_forced_exact_router_batch(name, T):
    """GMOE_FLAG_EXACT_ROUTER on a batch: every token replays glm.c's fp32 chains (in the
    batch router's last kernel, or k_router_tok for more than 64 experts)."""
    shape = {"small": SMALL, "glm": gmoe.GLM47_FLASH, "wide": WIDE}[name]
    want, got, st, stats = run_case(shape, seed=8, T=T, flags=gmoe.GMOE_FLAG_EXACT_ROUTER)
    check(want, got, st, stats)
    # the replay is glm.c's fp32 chain with libm's expf bits: probabilities and weights are
    # the reference's bit for bit
    assert np.array_equal(st["router_prob"].view(np.uint32), want["router_prob"].view(np.uint32)), "router_prob bits"
    assert np.array_equal(st["topk_w"].view(np.uint32), want["topk_w"].view(np.uint32)), "topk_w bits"
    assert stats["routing_exact_path"] >= T


def lists_from_topk(topk, E):
    """Brute-force per-expert lists: expert e's tokens in ascending order."""
    offs, toks = [0], []
    for e in range(E):
        toks += [t for t in range(topk.shape[0]) if e in topk[t]]
        offs.append(len(toks))
    return np.array(offs, np.int32), np.array(toks, np.int32)


# seed 12 of the 256-expert case holds an exact tie among one token's top K+1 scores,
# which the exact replay must break as glm.c does (the lower expert index first)
@pytest.mark.parametrize("name,T,seed", [("small", 200, 12), ("small", 33, 12), ("widest", 45, 12),
                                         ("widest", 45, 17)])
def test_ragged_batch_lists(name, T, seed):
    """Batches that are no multiple of the GEMM tile (32 rows): experts with two
    tiles, the second partial (16 experts, T=200), and many empty or single-row lists
    (256 experts, T=45). The per-expert lists equal a brute-force grouping of the
    oracle's top-k, and the layer's outputs the oracle's."""
    shape = {"small": SMALL, "widest": WIDEST}[name]
    want, got, st, stats = run_case(shape, seed=seed, T=T, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    check(want, got, st, stats)
    offs, toks = lists_from_topk(want["topk_idx"], shape.E)
    np.testing.assert_array_equal(st["expert_offsets"], offs, err_msg="per-expert offsets")
    np.testing.assert_array_equal(st["expert_tokens"], toks, err_msg="per-expert token lists")
