"""Full-size parity on the GPU against the golden fixtures written by glm.c's own
infer.c (tests/golden/make_golden.py): the GLM-4.7-Flash layer at T=1, and
batches of T=128 (Zipf-skewed routing) and T=512 tokens, each token being an
independent decode step of the reference (infer.c:2190-2233).

Bar: top-k indices and the per-expert token lists exact; xn bit-identical; float
outputs within max-abs 1e-2 and rel-L2 1e-3 (router probabilities and weights
within 1e-5). The batches are also compared row by row, all T rows, with the oracle
run on the same tokens."""
import numpy as np
import pytest

import gmoe
import oracle
from conftest import assert_close
from golden_data import load

pytestmark = pytest.mark.gpu

S = gmoe.GLM47_FLASH


@pytest.fixture(scope="module")
def layers():
    """Slot 1: seed-0 layer 1 with N(0, 0.01) bias; slot 2: the same layer with Zipf bias."""
    return {1: gmoe.HostLayer(S, seed=0, layer=1), 2: gmoe.HostLayer(S, seed=0, layer=1, bias_mode=gmoe.SYNTH_BIAS_ZIPF)}


@pytest.fixture(scope="module")
def ctx(layers):
    print("[setup] GLM-4.7-Flash layer 1, normal and Zipf bias, max_tokens 512", flush=True)
    c = gmoe.Context(S, n_layers=3, max_tokens=512)
    for slot, hl in layers.items():
        c.upload(slot, hl)
    yield c
    c.close()


def test_glm_t1(ctx):
    g = load("glm_t1")
    print("[case] glm_t1 T=1", flush=True)
    got, st = gmoe.forward_host(ctx, 1, g["x"])
    np.testing.assert_array_equal(st["topk_idx"], g["topk_idx"], err_msg="top-k indices")
    assert np.array_equal(st["xn"].view(np.uint32), g["xn"].view(np.uint32)), "xn not bit-identical"
    assert_close(st["router_prob"], g["router_prob"], "router_prob", max_abs=1e-5, rel_l2=1e-5)
    assert_close(st["topk_w"], g["topk_w"], "topk_w", max_abs=1e-5, rel_l2=1e-5)
    assert_close(st["shared_out"], g["shared_out"], "shared_out")
    assert_close(st["routed_out"], g["routed_out"], "routed_out")
    assert_close(got, g["x_out"], "x_out")


@pytest.mark.parametrize("name,slot,T,stream", [("dispatch_t128_zipf", 2, 128, 1), ("dispatch_t512", 1, 512, 2)])
def test_batched_tokens(ctx, layers, name, slot, T, stream):
    g = load(name)
    print(f"[case] {name} T={T}", flush=True)
    x = gmoe.activations(0, stream, T, S.D)
    assert np.array_equal(x[g["rows"]], g["x_rows"]), "input generator drifted from the fixture"
    got, st = gmoe.forward_host(ctx, slot, x)
    np.testing.assert_array_equal(st["topk_idx"], g["topk_idx"], err_msg="top-k indices")
    assert_close(st["topk_w"], g["topk_w"], "topk_w", max_abs=1e-5, rel_l2=1e-5)
    np.testing.assert_array_equal(st["expert_offsets"], g["offsets"], err_msg="per-expert offsets")
    np.testing.assert_array_equal(st["expert_tokens"], g["tokens"], err_msg="per-expert token lists")
    assert_close(got[g["rows"]], g["x_out_rows"], "sampled x_out rows")
    assert_close(got.astype(np.float64).sum(axis=1), g["x_out_row_sums"], "x_out row sums", max_abs=0.1)
    sumsq = float((got.astype(np.float64) ** 2).sum())
    assert abs(sumsq / float(g["x_out_sumsq"]) - 1) < 1e-5
    # every row against the oracle (the fixture stores six): each token is its own decode step
    want = oracle.Oracle("port").layer(S, layers[slot], x)
    np.testing.assert_array_equal(want["topk_idx"], g["topk_idx"], err_msg="oracle vs fixture top-k")
    for what in ("shared_out", "routed_out"):
        assert_close(st[what], want[what], f"all rows {what}")
    assert_close(got, want["x_out"], "all rows x_out")
    row_err = np.abs(got.astype(np.float64) - want["x_out"]).max(axis=1)
    assert row_err.max() <= 1e-2, f"row {int(row_err.argmax())} max-abs {row_err.max():.3e}"
