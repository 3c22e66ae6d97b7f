"""glm.c's own token forward on a checkpoint file (ref_decode in oracle/ref_harness.c:
infer.c's runtime_open, runstate_build, glm_cpu_forward_token_dual_checkpoints and
glm_cpu_forward_token, compiled from the reference sources into oracle/_ref), run in a
child process because glm.c's loader exits the process on a file it rejects.

reference_decode returns, for tokens[i] fed at position i (teacher-forced), x after each
layer's attention and after its FFN ([n][n_layers][dim]) and the logits ([n][vocab])."""
import os
import subprocess
import sys

import numpy as np

import oracle

SCRIPT = r"""
import ctypes as C, sys
import numpy as np
lib = C.CDLL(sys.argv[1])
FP = C.POINTER(C.c_float)
lib.ref_decode.argtypes = [C.c_char_p, C.POINTER(C.c_int), C.c_int, C.c_int, FP, FP, FP]
lib.ref_decode.restype = C.c_int
path, d = sys.argv[2], sys.argv[3]
cap, L, D, V = (int(v) for v in sys.argv[4:8])
tokens = np.load(d + "/tokens.npy").astype(np.int32)
n = len(tokens)
attn = np.zeros((n, L, D), np.float32)
layer = np.zeros((n, L, D), np.float32)
logits = np.zeros((n, V), np.float32)
rc = lib.ref_decode(path.encode(), tokens.ctypes.data_as(C.POINTER(C.c_int)), n, cap, attn.ctypes.data_as(FP),
                    layer.ctypes.data_as(FP), logits.ctypes.data_as(FP))
assert rc == 0, rc
np.save(d + "/attn.npy", attn)
np.save(d + "/layer.npy", layer)
np.save(d + "/logits.npy", logits)
print("ok")
"""


def available():
    return oracle.available("reference")


def reference_decode(path, tokens, cache_cap, n_layers, dim, vocab, work_dir):
    work_dir = str(work_dir)
    os.makedirs(work_dir, exist_ok=True)
    np.save(os.path.join(work_dir, "tokens.npy"), np.asarray(tokens, np.int32))
    args = [sys.executable, "-c", SCRIPT, oracle.PATHS["reference"], str(path), work_dir, str(cache_cap),
            str(n_layers), str(dim), str(vocab)]
    r = subprocess.run(args, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, f"glm.c's forward failed: {r.stdout} {r.stderr}"
    return {k: np.load(os.path.join(work_dir, f"{k}.npy")) for k in ("attn", "layer", "logits")}
