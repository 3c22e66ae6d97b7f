"""The rule by which the batch router's exact replay is restricted to a subset of the
experts (router.h, exact_router_subset), checked on the CPU against glm.c's insertion
top-k (infer.c:1110-1135: value descending, ties to the lower index, -inf never chosen).

Each expert's exact selection score lies in a certified interval [lo, hi]. With L the
K-th largest lo, at least K experts score at least L, so an expert with hi < L is never
among the K best; U = {e : hi >= L} is replayed and everything else is set to -inf. The
rule must leave glm.c's top-k (experts and order) unchanged for random, tied, clustered
and uncertified (NaN: lo = -inf, hi = +inf) intervals. Two plausible slips of the rule
(a strict hi > L, and L taken from the upper ends) are planted here and must be caught."""
import numpy as np


def glm_topk(sel, K):
    order = sorted(range(len(sel)), key=lambda e: (-sel[e], e))
    return [e for e in order[:K] if sel[e] > -np.inf]


def subset(lo, hi, K, strict=False, from_hi=False):
    ends = hi if from_hi else lo
    L = np.sort(ends)[::-1][K - 1]
    return [e for e in range(len(lo)) if (hi[e] > L if strict else hi[e] >= L)]


def cases(n, seed):
    rng = np.random.default_rng(seed)
    for trial in range(n):
        E = int(rng.choice([8, 16, 64, 128, 256]))
        K = int(rng.integers(1, min(8, E) + 1))
        mode = trial % 5
        exact = rng.standard_normal(E).astype(np.float32)
        if mode == 1:  # exact ties, some at the cut
            exact[rng.integers(0, E, E // 2)] = exact[0]
        if mode == 2:  # clustered near the cut
            exact = (rng.integers(0, 5, E) * 1e-3).astype(np.float32)
        half = np.abs(rng.standard_normal(E)).astype(np.float32) * np.float32(10 ** rng.uniform(-6, -1))
        lo = exact - half * rng.uniform(0, 1, E).astype(np.float32)
        hi = exact + half * rng.uniform(0, 1, E).astype(np.float32)
        if mode == 3:  # an uncertified expert
            j = rng.integers(0, E)
            lo[j], hi[j] = -np.inf, np.inf
        if mode == 4:  # zero-width intervals: the scores themselves, with ties
            exact[rng.integers(0, E, E // 2)] = exact[1]
            lo, hi = exact.copy(), exact.copy()
        yield exact, lo, hi, K


def mismatches(n, seed, **kw):
    bad = 0
    for exact, lo, hi, K in cases(n, seed):
        U = subset(lo, hi, K, **kw)
        sel_u = np.full(len(exact), -np.inf, np.float32)
        sel_u[U] = exact[U]
        bad += glm_topk(sel_u, K) != glm_topk(exact, K)
    return bad


def test_subset_keeps_glms_topk():
    assert mismatches(4000, 0) == 0


def test_planted_slips_are_caught():
    assert mismatches(4000, 0, strict=True) > 0
    assert mismatches(4000, 0, from_hi=True) > 0
