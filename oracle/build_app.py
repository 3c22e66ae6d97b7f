"""ORACLE build recipe -- test infrastructure only.

Builds glm.c's own command-line app twice from the reference sources where they lie
(REF_DIR), into oracle/_ref/ only:

  _ref/glm-cpu   main.c + infer.c + backend.c as the reference Makefile builds them
                 (Makefile:1-2, 89: -O3 -D_FILE_OFFSET_BITS=64 -fopenmp; no BLAS)
  _ref/glm-hip   the same app with the drop-in patch that INTEGRATION.md section 1 gives
                 (--backend hip, GLM_BACKEND=hip, the MoE hook, batched prefill), linked
                 against glm.c_amd/libglm_hip.so in place of backend.c

The patched copies of the sources live in a temporary directory that is deleted after the
compile: no reference source is written into the repository or travels with it. Each edit
is anchored on one statement of the reference; the script fails if an anchor is not found
exactly once (that is, if the reference changed under the patch).

    python3 oracle/build_app.py [REF_DIR]
"""
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG = os.path.join(ROOT, "glm.c_amd")
OUT = os.path.join(HERE, "_ref")
CFLAGS = ["-O3", "-D_FILE_OFFSET_BITS=64", "-fopenmp"]

# (file, anchor, replacement, count): the anchor must occur `count` times (0: at least once)
EDITS = [
    # model.h:161-164: one more backend
    ("model.h", "    BACKEND_METAL = 1,\n", "    BACKEND_METAL = 1,\n    BACKEND_HIP = 2,\n", 1),
    # backend.h: the MoE hook and the batched prompt prefill of libglm_hip.so
    ("backend.h", "int glm_backend_try_metal_matvec(",
     "int glm_backend_try_hip_moe(const Runtime *rt, RunState *st, int layer_idx, int debug_mode);\n"
     "int glm_hip_prefill(const Runtime *rt, RunState *st, const int *tokens, int n, int pos0, int debug_mode);\n"
     "int glm_backend_try_metal_matvec(", 1),
    # infer.c:1087: the MoE layer offload, first statement of apply_moe_shared_ffn_layer
    ("infer.c",
     "static void apply_moe_shared_ffn_layer(const Runtime *rt, RunState *s, int gs, int layer_idx, int debug_mode, int pos) {\n",
     "static void apply_moe_shared_ffn_layer(const Runtime *rt, RunState *s, int gs, int layer_idx, int debug_mode, int pos) {\n"
     "    if (glm_backend_try_hip_moe(rt, s, layer_idx, debug_mode) == 0) return;\n", 1),
    # infer.c:2029-2041: --backend hip
    ("infer.c",
     "            } else if (strcmp(v, \"metal\") == 0) {\n                backend = BACKEND_METAL;\n"
     "                backend_set = 1;\n            }",
     "            } else if (strcmp(v, \"metal\") == 0) {\n                backend = BACKEND_METAL;\n"
     "                backend_set = 1;\n            } else if (strcmp(v, \"hip\") == 0) {\n"
     "                backend = BACKEND_HIP;\n                backend_set = 1;\n            }", 1),
    # infer.c:2047-2050: GLM_BACKEND=hip
    ("infer.c", "if (env_backend && strcmp(env_backend, \"metal\") == 0) backend = BACKEND_METAL;",
     "if (env_backend && strcmp(env_backend, \"metal\") == 0) backend = BACKEND_METAL;\n"
     "        if (env_backend && strcmp(env_backend, \"hip\") == 0) backend = BACKEND_HIP;", 1),
    # infer.c:2178-2190: the prompt (all but its last token) by batched prefill, then the loop
    # runs the last prompt token as before
    ("infer.c", "    int prompt_index = 1;\n",
     "    int prompt_index = 1;\n"
     "    int pos_begin = 0;\n"
     "    if (use_metal == BACKEND_HIP && n_prompt > 1 && bench_mode == BENCH_MODE_OFF) {\n"
     "        if (glm_hip_prefill(&rt, &st, prompt_ids, n_prompt - 1, 0, debug_mode) != 0) die(\"prefill failed\");\n"
     "        pos_begin = n_prompt - 1;\n"
     "        token = prompt_ids[n_prompt - 1];\n"
     "        if (token < 0 || token >= rt.cfg.vocab_size) token = 0;\n"
     "        prompt_index = n_prompt;\n"
     "    }\n", 1),
    ("infer.c", "    for (int pos = 0; pos < cache_cap; pos++) {\n        if (bench_mode == BENCH_MODE_PREFILL",
     "    for (int pos = pos_begin; pos < cache_cap; pos++) {\n        if (bench_mode == BENCH_MODE_PREFILL", 1),
    # the backend's name in the banner and the bench report
    ("infer.c", "backend == BACKEND_METAL ? \"metal\" : \"cpu\"",
     "backend == BACKEND_METAL ? \"metal\" : backend == BACKEND_HIP ? \"hip\" : \"cpu\"", 0),
]


def patch(src_dir, dst_dir):
    for name in ("main.c", "infer.c", "model.h", "backend.h"):
        shutil.copy(os.path.join(src_dir, name), os.path.join(dst_dir, name))
    for name, anchor, repl, count in EDITS:
        path = os.path.join(dst_dir, name)
        with open(path) as f:
            text = f.read()
        n = text.count(anchor)
        if n == 0 or (count and n != count):
            raise SystemExit(f"build_app: anchor found {n} times in {name}: {anchor[:60]!r}")
        with open(path, "w") as f:
            f.write(text.replace(anchor, repl))


def cc(args):
    cmd = [os.environ.get("CC", "cc")] + CFLAGS + args
    print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    os.makedirs(OUT, exist_ok=True)
    cc(["-o", os.path.join(OUT, "glm-cpu")] + [os.path.join(ref, f) for f in ("main.c", "infer.c", "backend.c")]
       + ["-lm"])
    tmp = tempfile.mkdtemp(prefix="glm_app_")
    try:
        patch(ref, tmp)
        # libglm_hip.so through an rpath relative to the binary, so that the pair travels
        cc(["-I" + tmp, "-o", os.path.join(OUT, "glm-hip"), os.path.join(tmp, "main.c"), os.path.join(tmp, "infer.c"),
            "-L" + PKG, "-lglm_hip", "-lgmoe", "-Wl,-rpath,$ORIGIN/../../glm.c_amd", "-lm"])
    finally:
        shutil.rmtree(tmp)


if __name__ == "__main__":
    main()
