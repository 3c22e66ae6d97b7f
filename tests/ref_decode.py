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


STAGE_SCRIPT = r"""
import ctypes as C, sys
import numpy as np
lib = C.CDLL(sys.argv[1])
FP = C.POINTER(C.c_float)
path, d, what = sys.argv[2], sys.argv[3], sys.argv[4]
a = dict(np.load(d + "/args.npz"))
if what == "stage":
    lib.ref_stage.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_int, FP, FP, FP, FP]
    lib.ref_stage.restype = C.c_int
    out = np.zeros(int(a["n_out"]), np.float32)
    def fp(k):
        return a[k].ctypes.data_as(FP) if k in a else None
    rc = lib.ref_stage(path.encode(), int(a["stage"]), int(a["layer"]), int(a["token"]), int(a["pos"]), fp("comp"),
                       fp("pe"), fp("x_in"), out.ctypes.data_as(FP))
    assert rc == 0, rc
    np.save(d + "/out.npy", out)
else:
    L, D, V = int(a["L"]), int(a["D"]), int(a["V"])
    lib.ref_forward_zero_cache.argtypes = [C.c_char_p, C.c_int, C.c_int, FP, FP, FP]
    lib.ref_forward_zero_cache.restype = C.c_int
    attn = np.zeros((L, D), np.float32)
    layer = np.zeros((L, D), np.float32)
    logits = np.zeros(V, np.float32)
    rc = lib.ref_forward_zero_cache(path.encode(), int(a["token"]), int(a["pos"]), attn.ctypes.data_as(FP),
                                    layer.ctypes.data_as(FP), logits.ctypes.data_as(FP))
    assert rc == 0, rc
    np.savez(d + "/out.npz", attn=attn, layer=layer, logits=logits)
print("ok")
"""


def _child(path, work_dir, what, args):
    work_dir = str(work_dir)
    os.makedirs(work_dir, exist_ok=True)
    np.savez(os.path.join(work_dir, "args.npz"), **args)
    r = subprocess.run([sys.executable, "-c", STAGE_SCRIPT, oracle.PATHS["reference"], str(path), work_dir, what],
                       capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, f"glm.c's {what} failed: {r.stdout} {r.stderr}"


def reference_stage(path, work_dir, stage, layer, pos, n_out, token=0, x_in=None, comp=None, pe=None):
    """glm.c's own step (ref_stage in oracle/ref_harness.c) on the given inputs: stage 0 layer
    `layer`'s attention at pos over cache rows comp/pe (x_in None: the token's embedding),
    1 its FFN, 2 the final norm and LM head. Returns the n_out outputs."""
    args = {"stage": np.int32(stage), "layer": np.int32(layer), "token": np.int32(token), "pos": np.int32(pos),
            "n_out": np.int64(n_out)}
    for k, v in (("x_in", x_in), ("comp", comp), ("pe", pe)):
        if v is not None:
            args[k] = np.ascontiguousarray(v, np.float32).ravel()
    _child(path, work_dir, "stage", args)
    return np.load(os.path.join(str(work_dir), "out.npy"))


def reference_zero_cache(path, work_dir, token, pos, n_layers, dim, vocab):
    """glm.c's forward of `token` at pos over runstate_build's zeroed cache: dual checkpoints
    and logits (ref_forward_zero_cache)."""
    _child(path, work_dir, "zero", {"token": np.int32(token), "pos": np.int32(pos), "L": np.int32(n_layers),
                                    "D": np.int32(dim), "V": np.int32(vocab)})
    out = np.load(os.path.join(str(work_dir), "out.npz"))
    return {k: out[k] for k in ("attn", "layer", "logits")}
