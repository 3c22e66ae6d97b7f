"""The router's device expf against the C library's, over every one of the 2^32 fp32 inputs.

glm.c's sigmoid is 1 / (1 + expf(-logit)) with libm's expf (infer.c:1105), and its top-k
orders experts by the resulting scores with a strict `>` (infer.c:1110-1135). The exact
router replay therefore evaluates libm's expf bit for bit (expf_exact.h); the ends of a
certified selection interval use the GPU's fast expf and are widened for up to 2 ulp of
difference from libm. Both claims are checked exhaustively here (about 30 s)."""
import ctypes as C

import numpy as np
import pytest

import gmoe
import oracle

pytestmark = pytest.mark.gpu

CHUNK = 1 << 26


def sweep(which, max_ulp):
    lib = gmoe.gmoe_lib()
    hip = gmoe.hip()
    dev = gmoe.DeviceArray(CHUNK * 4)
    host = np.empty(CHUNK, np.float32)
    bad, first_bad = 0, -1
    for c in range((1 << 32) // CHUNK):
        first = c * CHUNK
        gmoe.check(lib.gmoe_expf_eval(first, CHUNK, which, dev.ptr, None), "gmoe_expf_eval")
        gmoe.hip_check(hip.hipMemcpy(host.ctypes.data_as(C.c_void_p), dev.ptr, CHUNK * 4, gmoe.HIP_D2H), "hipMemcpy")
        n, where = oracle.expf_compare(first, host, max_ulp)
        if n and first_bad < 0:
            first_bad = where
        bad += n
        if c % 16 == 15:
            print(f"[expf which={which}] inputs up to 0x{first + CHUNK - 1:08x}: {bad} beyond {max_ulp} ulp", flush=True)
    dev.free()
    return bad, first_bad


def test_exact_expf_equals_libm_on_every_input():
    bad, first_bad = sweep(0, 0)
    x = np.uint32(first_bad if first_bad >= 0 else 0).view(np.float32)
    assert bad == 0, f"{bad} inputs differ from libm's expf, the first at bits 0x{first_bad:08x} (x={x!r})"


def test_fast_expf_within_two_ulp_of_libm():
    bad, first_bad = sweep(1, 2)
    assert bad == 0, f"{bad} inputs beyond 2 ulp of libm, the first at bits 0x{first_bad:08x}"


def test_context_reports_the_glibc_the_table_was_measured_against():
    """The exception table records the glibc it was measured against; a context compares it
    with the running process's glibc and reports the match in its stats (this image's
    glibc is the one the committed table was measured on)."""
    ctx = gmoe.Context(gmoe.GLM47_FLASH, n_layers=2, max_tokens=1, device=0)
    try:
        assert ctx.stats()["expf_libc_match"] == 1
    finally:
        ctx.close()
