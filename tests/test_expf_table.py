"""The exception table behind the GPU's libm-exact expf (glm.c_amd/data/expf_exceptions.bin).

glm.c's router sigmoid calls the C library's expf (infer.c:1105) and its top-k orders
experts by the result's last bit when scores tie that closely (infer.c:1110-1135). The
GPU rounds an accurate double exp to fp32 and consults this table for the inputs where
libm rounds the other way, or where two accurate doubles could round differently. These
tests re-measure the table over every fp32 input against this machine's libm and check
the committed file is exactly that, and check its format and premises."""
import os
import struct
import subprocess
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "glm.c_amd")
TABLE = os.path.join(PKG, "data", "expf_exceptions.bin")
TOOL = os.path.join(PKG, "_build", "expf_table")


def read_table(path):
    raw = open(path, "rb").read()
    assert raw[:8] == b"GMEXPF02"
    n, near = struct.unpack_from("<II", raw, 8)
    libc = raw[16:32].rstrip(b"\0").decode()
    keys = np.frombuffer(raw, "<u4", n, 32)
    nw = (n + 31) // 32
    bits = np.frombuffer(raw, "<u4", nw, 32 + 4 * n)
    assert len(raw) == 32 + 4 * n + 4 * nw
    up = (bits[np.arange(n) // 32] >> (np.arange(n) % 32).astype(np.uint32)) & 1
    return keys, up.astype(bool), near, libc


def this_libc():
    import ctypes

    libc = ctypes.CDLL("libc.so.6")
    libc.gnu_get_libc_version.restype = ctypes.c_char_p
    return libc.gnu_get_libc_version().decode()


def test_table_format_and_premises():
    keys, up, near, libc = read_table(TABLE)
    assert near == 7
    assert libc == this_libc(), "the table records the glibc it was measured against"
    assert keys.size > 100000
    assert np.all(np.diff(keys.astype(np.int64)) > 0), "keys must ascend"
    x = keys.view(np.float32)
    assert np.all(np.isfinite(x))
    # only inputs whose exp is a normal or subnormal float need an entry
    assert x.min() > -104.0 and x.max() < 89.0
    # the recorded neighbour is what libm returns (spot check through the C library)
    import ctypes

    libm = ctypes.CDLL("libm.so.6")
    libm.expf.argtypes = [ctypes.c_float]
    libm.expf.restype = ctypes.c_float
    libm.exp.argtypes = [ctypes.c_double]
    libm.exp.restype = ctypes.c_double
    rng = np.random.default_rng(0)
    for i in rng.choice(keys.size, 400, replace=False):
        xi = float(x[i])
        d = libm.exp(xi)
        g = np.float32(libm.expf(np.float32(xi)))
        m, ex = np.frexp(d)
        ue = max(int(ex) - 24, -149)
        fl = np.floor(np.ldexp(d, -ue))
        pick = np.float32(np.ldexp(fl + 1.0 if up[i] else fl, ue))
        assert g.view(np.uint32) == pick.view(np.uint32), f"entry {i} (x={xi!r})"


def test_committed_table_is_this_libm_measured_over_every_input():
    assert os.path.exists(TOOL), "build first (make -C glm.c_amd all builds the sweep tool)"
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "t.bin")
        r = subprocess.run([TOOL, "sweep", out], capture_output=True, text=True, timeout=600)
        assert r.returncode == 0, r.stderr + r.stdout
        assert "0 inputs outside the model" in r.stdout
        assert open(out, "rb").read() == open(TABLE, "rb").read(), "data/expf_exceptions.bin differs from a fresh sweep"
