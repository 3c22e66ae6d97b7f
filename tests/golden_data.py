"""Access to the committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from glm.c's own infer.c) and the shapes and input
edits they were made with."""
import os

import numpy as np

import gmoe

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SMALL = gmoe.Shape(dim=256, moe_ffn_dim=256, n_routed_experts=16, n_experts_used=4)


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def with_ties_and_nan(hl):
    """Expert 5 duplicates expert 3 (equal logits and bias: an exact tie in sel, lifted to
    the top of the ranking); expert 9 gets a NaN router row, so its probability is NaN."""
    hl.gate_inp[5] = hl.gate_inp[3]
    hl.exp_probs_b[5] = hl.exp_probs_b[3]
    hl.gate_inp[9] = np.nan
    hl.exp_probs_b[3] += 0.5
    hl.exp_probs_b[5] += 0.5
    return hl


def digests(g):
    return dict(zip(g["digest_keys"].tolist(), g["digest_values"].tolist()))
