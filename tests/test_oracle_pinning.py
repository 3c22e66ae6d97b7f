"""Each function of the CPU restatement pinned by what the mathematics fixes,
independently of glm.c's build: closed forms, brute force on small inputs, fp64
recomputation with an error bound, and invariants. Each check is chosen so that
a plausible slip (a dropped term, float instead of double accumulation, a
transposed operand, a wrong tie rule, the wrong gate of SwiGLU) fails it.
"""
import ctypes as C
import zlib

import numpy as np
import pytest

import gmoe
import oracle

from golden_data import SMALL

F32 = np.float32


@pytest.fixture(scope="module")
def lib():
    return oracle.Oracle("port").lib


def p(a):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- rmsnorm (infer.c:746-752)

def rmsnorm_closed_form(x, w, eps=F32(1e-5)):
    ss = np.cumsum(x.astype(np.float64) ** 2)[-1]  # sequential double sum
    mean = F32(ss / len(x))
    scale = F32(1.0) / np.sqrt(F32(mean + eps))
    return (x * scale).astype(F32) * w


@pytest.mark.parametrize("case", ["normal", "wide_range", "tiny"])
def test_rmsnorm_closed_form(lib, case):
    rng = np.random.default_rng(1)
    n = 2048
    x = rng.standard_normal(n).astype(F32)
    if case == "wide_range":  # float accumulation of the squares would lose the small terms
        x[::7] *= F32(3e3)
    if case == "tiny":  # eps dominates the mean
        x *= F32(1e-4)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(F32)
    out = np.zeros(n, F32)
    lib.oracle_rmsnorm(p(out), p(x), p(w), n)
    assert np.array_equal(out.view(np.uint32), rmsnorm_closed_form(x, w).view(np.uint32))


def test_rmsnorm_unit_rms(lib):
    x = np.random.default_rng(2).standard_normal(4096).astype(F32) * F32(17.0)
    w = np.ones_like(x)
    out = np.zeros_like(x)
    lib.oracle_rmsnorm(p(out), p(x), p(w), len(x))
    assert abs(float(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 1e-4


# ---------------------------------------------------------------- Q8_0 matvec (infer.c:765-786)

@pytest.mark.parametrize("rows,cols", [(64, 256), (96, 2048), (40, 1536)])
def test_matvec_q8_against_fp64_dequantised(lib, rows, cols):
    rng = np.random.default_rng(rows + cols)
    gs = 32
    q = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    s = (np.abs(rng.standard_normal((rows, cols // gs))) * 0.002).astype(F32)
    x = rng.standard_normal(cols).astype(F32)
    y = np.zeros(rows, F32)
    lib.oracle_matvec_q8(p(q), p(s), p(x), p(y), rows, cols, gs)
    W = q.astype(np.float64) * np.repeat(s.astype(np.float64), gs, axis=1)
    y64 = W @ x.astype(np.float64)
    mag = np.abs(W) @ np.abs(x.astype(np.float64))
    assert np.max(np.abs(y - y64) / mag) < 1e-5


# ---------------------------------------------------------------- router (infer.c:916-938)

def test_router_logits_are_one_sequential_fp32_chain(lib):
    rng = np.random.default_rng(3)
    E, D = 5, 256
    g = (rng.standard_normal((E, D)) * 0.02).astype(F32)
    x = rng.standard_normal(D).astype(F32)
    out = np.zeros(E, F32)
    lib.oracle_router_logits(p(g), p(x), p(out), E, D)
    for e in range(E):
        acc = F32(0.0)
        for i in range(D):
            acc = F32(acc + F32(g[e, i] * x[i]))
        assert out[e].view(np.uint32) == acc.view(np.uint32)
        exact = float(np.dot(g[e].astype(np.float64), x.astype(np.float64)))
        bound = D * 2.0 ** -24 * float(np.abs(g[e].astype(np.float64)) @ np.abs(x.astype(np.float64)))
        assert abs(float(out[e]) - exact) <= bound


def ulps(a, b):
    a, b = np.float32(a), np.float32(b)
    ia = np.int64(a.view(np.int32))
    ib = np.int64(b.view(np.int32))
    ia = np.where(ia < 0, np.int64(-(2 ** 31)) - ia, ia)
    ib = np.where(ib < 0, np.int64(-(2 ** 31)) - ib, ib)
    return abs(int(ia - ib))


def test_sigmoid_and_silu(lib):
    # fp32 chain expf -> add -> divide: within a few ulps of the exact value
    for v in np.linspace(-30, 30, 601).astype(F32):
        v64 = float(v)
        s = lib.oracle_sigmoid(v64)
        assert ulps(s, F32(1.0 / (1.0 + np.exp(-v64)))) <= 3, v
        si = lib.oracle_silu(v64)
        assert ulps(si, F32(v64 / (1.0 + np.exp(-v64)))) <= 3, v
    assert lib.oracle_sigmoid(0.0) == 0.5
    assert lib.oracle_sigmoid(float("inf")) == 1.0
    assert lib.oracle_sigmoid(float("-inf")) == 0.0
    assert np.isnan(lib.oracle_sigmoid(float("nan")))
    assert lib.oracle_silu(0.0) == 0.0


# ---------------------------------------------------------------- top-k + normalisation (infer.c:1108-1145)

def topk_brute_force(prob, bias, K):
    """Stable sort by sel descending (ties: lower index first); NaN and -inf never qualify."""
    sel = (prob + bias).astype(F32)
    cand = [e for e in range(len(prob)) if sel[e] > -np.inf]
    cand.sort(key=lambda e: -float(sel[e]))
    idx = cand[:K] + [-1] * max(0, K - len(cand))
    w = np.array([prob[e] if e >= 0 else F32(-1e30) for e in idx], F32)
    total = F32(0.0)
    for k, e in enumerate(idx):
        if e >= 0:
            total = F32(total + w[k])
    if total > 0:
        inv = F32(1.0) / max(total, F32(6.103515625e-5))
        w = (w * inv).astype(F32)
    return np.array(idx, np.int32), w


def run_topk(lib, prob, bias, K):
    idx = np.zeros(K, np.int32)
    w = np.zeros(K, F32)
    lib.oracle_topk(p(prob), p(bias), len(prob), K, p(idx), p(w))
    return idx, w


@pytest.mark.parametrize("case", ["random", "ties", "nan", "few_experts", "tiny_probs", "all_zero", "neg_inf_bias"])
def test_topk_brute_force(lib, case):
    rng = np.random.default_rng(zlib.crc32(case.encode()))
    E, K = 16, 4
    for trial in range(50):
        prob = rng.random(E).astype(F32)
        bias = (rng.standard_normal(E) * 0.01).astype(F32)
        if case == "ties":
            prob[rng.integers(0, E, 6)] = prob[0]
            bias[:] = bias[0]
        if case == "nan":
            prob[rng.integers(0, E, 3)] = np.nan
        if case == "few_experts":
            E2 = int(rng.integers(1, K))
            prob, bias = prob[:E2].copy(), bias[:E2].copy()
        if case == "tiny_probs":
            prob *= F32(1e-6)
            bias[:] = 0
        if case == "all_zero":
            prob[:] = 0
        if case == "neg_inf_bias":
            bias[rng.integers(0, E, 5)] = -np.inf
        got_i, got_w = run_topk(lib, prob, bias, K)
        want_i, want_w = topk_brute_force(prob, bias, K)
        assert np.array_equal(got_i, want_i), (case, trial, got_i, want_i)
        assert np.array_equal(got_w.view(np.uint32), want_w.view(np.uint32)), (case, trial, got_w, want_w)


# ---------------------------------------------------------------- per-expert token lists

@pytest.mark.parametrize("T,E,K", [(0, 8, 2), (1, 64, 4), (37, 16, 4), (300, 64, 4)])
def test_dispatch_brute_force(T, E, K):
    rng = np.random.default_rng(T + E)
    topk = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32) if T else np.zeros((0, K), np.int32)
    if T > 3:
        topk[3, K - 1] = -1  # an empty slot (fewer experts than K) is skipped
    offsets, tokens, slots = oracle.dispatch(topk, E)
    pos = 0
    for e in range(E):
        want = [(t, k) for t in range(T) for k in range(K) if topk[t, k] == e]
        assert offsets[e] == pos
        got = list(zip(tokens[offsets[e]:offsets[e + 1]].tolist(), slots[offsets[e]:offsets[e + 1]].tolist()))
        assert got == want
        pos += len(want)
    assert offsets[E] == pos == len(tokens)


# ---------------------------------------------------------------- the composed layer (infer.c:1087-1216)

def dequant(q, s, gs=32):
    return q.astype(np.float64) * np.repeat(s.astype(np.float64), gs, axis=-1)


def swiglu_expert_fp64(xn, gq, gsc, uq, usc, dq, dsc):
    g = dequant(gq, gsc) @ xn
    u = dequant(uq, usc) @ xn
    h = g / (1.0 + np.exp(-g)) * u
    return dequant(dq, dsc) @ h


@pytest.fixture(scope="module")
def small_layer_run():
    hl = gmoe.HostLayer(SMALL, seed=21, layer=1, norm_mode=gmoe.SYNTH_NORM_RANDOM)
    x = gmoe.activations(21, 0, 3, SMALL.D)
    return hl, x, oracle.Oracle("port").layer(SMALL, hl, x)


def test_layer_residual_is_x_plus_shared_plus_routed(small_layer_run):
    hl, x, r = small_layer_run
    want = (x + (r["shared_out"] + r["routed_out"]).astype(F32)).astype(F32)
    assert np.array_equal(r["x_out"].view(np.uint32), want.view(np.uint32))


def test_layer_shared_expert_against_fp64(small_layer_run):
    hl, x, r = small_layer_run
    for t in range(x.shape[0]):
        xn = r["xn"][t].astype(np.float64)
        y = swiglu_expert_fp64(xn, hl.gate_sh_q, hl.gate_sh_s, hl.up_sh_q, hl.up_sh_s, hl.down_sh_q, hl.down_sh_s)
        assert np.linalg.norm(r["shared_out"][t] - y) <= 1e-5 * np.linalg.norm(y)


def test_layer_routed_experts_against_fp64(small_layer_run):
    hl, x, r = small_layer_run
    for t in range(x.shape[0]):
        xn = r["xn"][t].astype(np.float64)
        acc = np.zeros(SMALL.D)
        for k, e in enumerate(r["topk_idx"][t]):
            y = swiglu_expert_fp64(xn, hl.gate_q[e], hl.gate_s[e], hl.up_q[e], hl.up_s[e], hl.down_q[e], hl.down_s[e])
            acc += 1.8 * float(r["topk_w"][t, k]) * y
        assert np.linalg.norm(r["routed_out"][t] - acc) <= 1e-5 * np.linalg.norm(acc)
        # the weights are the unbiased probabilities of the chosen experts, normalised
        pw = r["router_prob"][t][r["topk_idx"][t]].astype(np.float64)
        assert np.allclose(r["topk_w"][t], pw / pw.sum(), rtol=1e-6)


def test_layer_routed_off(small_layer_run):
    hl, x, _ = small_layer_run
    r = oracle.Oracle("port").layer(SMALL, hl, x, disable_routed=True)
    assert not r["routed_out"].any()
    assert np.array_equal(r["x_out"], (x + r["shared_out"]).astype(F32))


def test_expf_compare_counts_bitwise_and_ulp_differences():
    """oracle_expf_compare, the checker of the GPU's expf, against numpy's bit patterns:
    a result one ulp off fails the bitwise comparison and passes at max_ulp=1; NaN
    matches NaN only."""
    import ctypes

    libm = ctypes.CDLL("libm.so.6")
    libm.expf.argtypes = [ctypes.c_float]
    libm.expf.restype = ctypes.c_float
    first = np.float32(-3.0).view(np.uint32)
    n = 4096
    xs = (np.uint32(first) + np.arange(n, dtype=np.uint32)).view(np.float32)
    exact = np.array([libm.expf(float(v)) for v in xs], np.float32)
    assert oracle.expf_compare(int(first), exact) == (0, -1)
    off = exact.copy()
    off[17] = np.nextafter(off[17], np.float32(np.inf))
    assert oracle.expf_compare(int(first), off) == (1, int(first) + 17)
    assert oracle.expf_compare(int(first), off, max_ulp=1) == (0, -1)
    nan_first = np.float32(np.nan).view(np.uint32)
    assert oracle.expf_compare(int(nan_first), np.array([np.nan], np.float32)) == (0, -1)
    assert oracle.expf_compare(int(nan_first), np.array([1.0], np.float32))[0] == 1
