"""The seeded synthetic-input generator (glm.c_amd/host/synth.c).

The benchmark workload and every fixture are defined by this generator, so it is
pinned three ways: element functions against numpy (fp16 rounding), statistical
shape of each draw, and the SHA-256 digests the golden fixtures recorded when
glm.c's own code produced their expected outputs.
"""
import numpy as np
import pytest

import gmoe

from golden_data import SMALL, digests, load


def test_fp16_rounding_matches_numpy():
    lib = gmoe.host_lib()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000) * 0.002,                    # the scale distribution
        rng.uniform(-65000, 65000, 5000),                      # normal range
        rng.uniform(-1e-4, 1e-4, 5000),                        # fp16 subnormals (< 6.1e-5)
        (np.arange(-2048, 2048) + 0.5) * 2.0 ** -14,           # exact halfway cases near the subnormal edge
        np.array([0.0, -0.0, 6.103515625e-05, 5.960464477539063e-08, 65504.0, 2.0 ** -25, 3 * 2.0 ** -26]),
    ]).astype(np.float32)
    got = np.array([lib.synth_round_fp16(float(v)) for v in vals], np.float32)
    want = vals.astype(np.float16).astype(np.float32)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} mismatches, first {vals[bad[0]]!r}: {got[bad[0]]!r} vs {want[bad[0]]!r}"


@pytest.fixture(scope="module")
def small_layer():
    return gmoe.HostLayer(SMALL, seed=3, layer=2, norm_mode=gmoe.SYNTH_NORM_RANDOM)


def test_q8_draws(small_layer):
    q = small_layer.gate_q.ravel()
    assert q.min() == -127 and q.max() == 127
    counts = np.bincount(q.astype(np.int64) + 127, minlength=255)
    assert counts.min() > 0.8 * counts.mean() and counts.max() < 1.2 * counts.mean()


def test_scales_are_fp16_exact_and_shaped(small_layer):
    for n in ("gate_s", "up_s", "down_s", "gate_sh_s", "up_sh_s", "down_sh_s"):
        s = getattr(small_layer, n)
        assert (s >= 0).all()
        assert np.array_equal(s, s.astype(np.float16).astype(np.float32)), n
    s = small_layer.gate_s.astype(np.float64).ravel()
    # |N(0,1)| * 0.002 has mean 0.002 * sqrt(2 / pi)
    assert abs(s.mean() / (0.002 * np.sqrt(2 / np.pi)) - 1) < 0.02


def test_router_and_norm_draws(small_layer):
    g = small_layer.gate_inp.astype(np.float64)
    assert abs(g.std() / 0.02 - 1) < 0.02 and abs(g.mean()) < 1e-3
    w = small_layer.ffn_norm.astype(np.float64)
    assert abs(w.mean() - 1) < 0.02 and abs(w.std() / 0.1 - 1) < 0.15
    ones = gmoe.HostLayer(SMALL, seed=3, layer=2, routed=False)
    assert (ones.ffn_norm == 1.0).all()


def test_expert_subset_equals_full_generation(small_layer):
    part = gmoe.HostLayer(SMALL, seed=3, layer=2, experts=(5, 9), norm_mode=gmoe.SYNTH_NORM_RANDOM)
    for n in ("gate_q", "gate_s", "up_q", "up_s", "down_q", "down_s"):
        assert np.array_equal(getattr(part, n)[5:9], getattr(small_layer, n)[5:9]), n
        assert not getattr(part, n)[:5].any() and not getattr(part, n)[9:].any()
    for n in ("gate_inp", "exp_probs_b", "gate_sh_q", "down_sh_s"):
        assert np.array_equal(getattr(part, n), getattr(small_layer, n)), n


def test_layers_and_seeds_differ():
    a = gmoe.HostLayer(SMALL, seed=3, layer=2, routed=False)
    b = gmoe.HostLayer(SMALL, seed=3, layer=3, routed=False)
    c = gmoe.HostLayer(SMALL, seed=4, layer=2, routed=False)
    assert not np.array_equal(a.gate_sh_q, b.gate_sh_q) and not np.array_equal(a.gate_sh_q, c.gate_sh_q)


def test_activations():
    x = gmoe.activations(0, 0, 64, 2048).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    assert np.array_equal(gmoe.activations(0, 0, 64, 2048), gmoe.activations(0, 0, 64, 2048))
    assert not np.array_equal(gmoe.activations(0, 1, 1, 2048), gmoe.activations(0, 0, 1, 2048))


def test_zipf_bias_is_skewed():
    hl = gmoe.HostLayer(gmoe.GLM47_FLASH, seed=0, layer=1, bias_mode=gmoe.SYNTH_BIAS_ZIPF, routed=False)
    b = np.sort(hl.exp_probs_b.astype(np.float64))[::-1]
    # beta * -1.2 * ln(rank): the top expert leads the median one by about beta * 1.2 * ln 32
    assert b[0] - b[31] > 0.5 * gmoe.ZIPF_BETA * 1.2 * np.log(32)


def sha(a):
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_digests_of_small_fixture(small_layer):
    want = digests(load("small"))
    hl = gmoe.HostLayer(SMALL, seed=7, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    for k, v in want.items():
        if "[" in k:
            n, e = k[:-1].split("[")
            got = sha(getattr(hl, n)[int(e)])
        else:
            got = sha(getattr(hl, k))
        assert got == v, k


def test_digests_of_glm_fixture(glm_layer1):
    for k, v in digests(load("glm_t1")).items():
        if "[" in k:
            n, e = k[:-1].split("[")
            got = sha(getattr(glm_layer1, n)[int(e)])
        else:
            got = sha(getattr(glm_layer1, k))
        assert got == v, k
