"""The drop-in boundary without a GPU: the shared libraries load and export every
function their headers declare, the ctypes mirrors match the C struct layouts,
include/glm_model.h is layout-identical to glm.c's model.h, and argument
validation fails with GMOE_ERR_INVALID before any device call.
"""
import ctypes as C
import os
import re
import subprocess
import sys
import tempfile

import pytest

import gmoe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
REF_MODEL_H = "/root/reference/model.h"


def declared_functions(header, prefix):
    text = open(os.path.join(INC, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"\w*)\s*\(", text)))


def exported(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_libgmoe_exports_every_declared_function():
    names = declared_functions("gmoe.h", "gmoe_")
    assert len(names) >= 15
    missing = set(names) - exported(gmoe.LIBGMOE)
    assert not missing, f"libgmoe.so lacks {sorted(missing)}"
    lib = gmoe.gmoe_lib()
    for n in names:
        getattr(lib, n)


def test_libglm_hip_exports_the_backend_interface():
    names = declared_functions("glm_backend.h", "glm_")
    assert {"glm_backend_init", "glm_backend_forward_token", "glm_backend_free", "glm_hip_init"} <= set(names)
    missing = set(names) - exported(gmoe.LIBHOST)
    assert not missing, f"libglm_hip.so lacks {sorted(missing)}"


def compile_and_run(source, include_dirs, defines=()):
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "probe.c"), os.path.join(d, "probe")
        open(src, "w").write(source)
        cmd = ["gcc", "-std=c11", "-o", exe, src] + [f"-I{i}" for i in include_dirs] + list(defines)
        subprocess.run(cmd, check=True, capture_output=True, text=True)
        return subprocess.run([exe], check=True, capture_output=True, text=True).stdout


CTYPES_MIRRORS = {
    "gmoe_config": gmoe.GmoeConfig,
    "gmoe_layer_weights": gmoe.LayerWeights,
    "gmoe_layer_state": gmoe.GmoeLayerState,
    "gmoe_stats": gmoe.GmoeStats,
    "gmoe_kernel_times": gmoe.GmoeKernelTimes,
}


def test_ctypes_structs_match_the_c_header():
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "gmoe.h"', "int main(void) {"]
    for cname, cls in CTYPES_MIRRORS.items():
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["return 0; }"]
    out = compile_and_run("\n".join(lines), [INC])
    for line in out.splitlines():
        cname, field, val = line.split()
        cls = CTYPES_MIRRORS[cname]
        want = C.sizeof(cls) if field == "sizeof" else getattr(cls, field).offset
        assert int(val) == want, f"{cname}.{field}: C {val}, ctypes {want}"


def error_codes():
    text = open(os.path.join(INC, "gmoe.h")).read()
    return {m.group(1): int(m.group(2)) for m in re.finditer(r"#define (GMOE_\w+)\s+\(?(-?\d+)\)?", text)}


def test_error_codes_and_flags():
    codes = error_codes()
    assert codes["GMOE_OK"] == 0
    assert codes["GMOE_ERR_INVALID"] == -1 and codes["GMOE_ERR_HIP"] == -2
    assert codes["GMOE_ERR_NOMEM"] == -3 and codes["GMOE_ERR_SCALE"] == -4
    assert codes["GMOE_FLAG_NO_ROUTED"] == gmoe.GMOE_FLAG_NO_ROUTED


@pytest.mark.parametrize("fields,needle", [
    ({"dim": 100}, "multiples of 256"),
    ({"dim": 4096}, "multiples of 256"),
    ({"moe_ffn_dim": 0}, "multiples of 256"),
    ({"n_routed_experts": 300}, "n_routed_experts"),
    ({"n_experts_used": 9}, "n_experts_used"),
    ({"n_shared_experts": 2}, "shared expert"),
    ({"group_size": 16, "q8_form": gmoe.GMOE_Q8_TILED}, "tiled form needs group_size 32"),
    ({"group_size": 8}, "multiple of 16"),
    ({"group_size": 48}, "divides dim"),
    ({"q8_form": 7}, "q8_form"),
    ({"n_layers": 1}, "n_layers"),
    ({"max_tokens": 0}, "max_tokens"),
])
def test_create_rejects_bad_config_before_touching_a_device(fields, needle):
    lib = gmoe.gmoe_lib()
    s = gmoe.GLM47_FLASH
    cfg = gmoe.GmoeConfig(s.D, s.F, s.E, s.K, 1, s.gs, 48, 1, 1.8, 1e-5, gmoe.GMOE_Q8_AUTO)
    for field, value in fields.items():
        setattr(cfg, field, value)
    h = C.c_void_p(1)
    rc = lib.gmoe_create(C.byref(h), 0, C.byref(cfg))
    assert rc == -1
    assert h.value is None
    assert needle in gmoe.last_error()


def test_null_arguments_are_rejected():
    lib = gmoe.gmoe_lib()
    assert lib.gmoe_create(None, 0, None) == -1
    assert lib.gmoe_upload_layer(None, 1, None) == -1
    assert lib.gmoe_forward(None, 1, 1, None, None, 0, None) == -1
    assert lib.gmoe_forward_layers(None, 1, 1, 1, None, None, 0, None) == -1
    assert lib.gmoe_get_stats(None, None) == -1
    lib.gmoe_destroy(None)  # a no-op


MODEL_STRUCTS = ["RuntimeConfig", "LayerAttnWeights", "LayerMoeShared", "LayerMoeRouted", "Runtime", "RunState"]


def struct_fields(header_text, name):
    m = re.search(r"\{([^{}]*)\}\s*" + name + r"\s*;", header_text)
    body = re.sub(r"/\*.*?\*/|//[^\n]*", "", m.group(1))
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if decl:
            fields.append(re.findall(r"(\w+)\s*(?:\[[^\]]*\])?\s*$", decl)[0])
    return fields


def layout_probe(header_path, fields):
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{header_path}"', "int main(void) {"]
    for s, fl in fields.items():
        lines.append(f'printf("{s} sizeof %zu\\n", sizeof({s}));')
        for f in fl:
            lines.append(f'printf("{s} {f} %zu\\n", offsetof({s}, {f}));')
    lines.append("return 0; }")
    return "\n".join(lines)


@pytest.mark.skipif(not os.path.exists(REF_MODEL_H), reason="glm.c's model.h is not present on this machine")
def test_glm_model_h_is_layout_identical_to_the_reference():
    text = open(os.path.join(INC, "glm_model.h")).read()
    fields = {s: struct_fields(text, s) for s in MODEL_STRUCTS}
    ours = compile_and_run(layout_probe(os.path.join(INC, "glm_model.h"), fields), [INC])
    theirs = compile_and_run(layout_probe(REF_MODEL_H, fields), [os.path.dirname(REF_MODEL_H)])
    assert ours == theirs


def run_backend(snippet):
    """Run a C call sequence against libglm_hip.so in a child process (the backend exits on failure)."""
    code = ("import ctypes as C, sys\n"
            f"lib = C.CDLL({gmoe.LIBHOST!r}, mode=C.RTLD_GLOBAL)\n" + snippet)
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=60)


def test_backend_cpu_init_is_a_no_op():
    r = run_backend("print(lib.glm_backend_init(0, None, None)); lib.glm_backend_free(0)")
    assert r.returncode == 0 and r.stdout.strip() == "0"


def test_backend_metal_is_unavailable_and_exits():
    r = run_backend("lib.glm_backend_init(1, None, None); print('returned')")
    assert r.returncode == 1 and "returned" not in r.stdout
    assert "[glm-metal]" in r.stderr


def test_backend_matvec_offload_declines():
    r = run_backend("print(lib.glm_backend_try_metal_matvec(None, None, None, None, 64, 64, 32),"
                    " lib.glm_backend_metal_matvec_enabled())")
    assert r.returncode == 0 and r.stdout.split() == ["-1", "0"]


def test_glm_model_ctypes_mirror_matches_the_c_header():
    """glm.c_amd/glm_model.py (the Runtime/RunState the GPU backend tests and the benchmark
    build) has include/glm_model.h's layout, field for field."""
    import glm_model

    text = open(os.path.join(INC, "glm_model.h")).read()
    fields = {s: struct_fields(text, s) for s in MODEL_STRUCTS}
    for s, fl in fields.items():
        assert [n for n, _ in glm_model.STRUCTS[s]._fields_] == fl, f"{s}: field list differs from glm_model.h"
    out = compile_and_run(layout_probe(os.path.join(INC, "glm_model.h"), fields), [INC])
    for line in out.splitlines():
        sname, field, val = line.split()
        cls = glm_model.STRUCTS[sname]
        want = C.sizeof(cls) if field == "sizeof" else getattr(cls, field).offset
        assert int(val) == want, f"{sname}.{field}: C {val}, ctypes {want}"
