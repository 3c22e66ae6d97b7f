import contextlib
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("glm.c_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


# Parity bar for floating-point outputs (max-abs 1e-2 and rel-L2 1e-3, fp32 accumulation).
MAX_ABS = 1e-2
REL_L2 = 1e-3


def assert_close(got, want, what, max_abs=MAX_ABS, rel_l2=REL_L2):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    err = np.abs(got - want)
    denom = np.linalg.norm(want)
    rel = np.linalg.norm(got - want) / denom if denom > 0 else np.linalg.norm(got - want)
    assert err.max() <= max_abs, f"{what}: max-abs {err.max():.3e} > {max_abs} (at {np.unravel_index(err.argmax(), err.shape)})"
    assert rel <= rel_l2, f"{what}: rel-L2 {rel:.3e} > {rel_l2}"
    return err.max(), rel


# The persistent T=1 kernels, chosen when a context is created: k_moe_relay (the default,
# GMOE_DECODE_KERNEL=2 or unset) and k_moe_stack (0), its fallback.
DECODE_KERNELS = {"stack": "0", "relay": "2"}
DECODE_KERNEL_NAMES = {"stack": "k_moe_stack", "relay": "k_moe_relay"}
DEFAULT_DECODE_KERNEL = "relay"


def current_decode_kernel():
    """The persistent kernel that a context created now runs its T=1 launches on."""
    env = os.environ.get("GMOE_DECODE_KERNEL")
    for kind, val in DECODE_KERNELS.items():
        if env == val:
            return kind
    return DEFAULT_DECODE_KERNEL


@contextlib.contextmanager
def decode_kernel(kind):
    """Contexts created inside run their T=1 launches on `kind` (a key of DECODE_KERNELS)."""
    old = os.environ.get("GMOE_DECODE_KERNEL")
    os.environ["GMOE_DECODE_KERNEL"] = DECODE_KERNELS[kind]
    try:
        yield
    finally:
        if old is None:
            os.environ.pop("GMOE_DECODE_KERNEL", None)
        else:
            os.environ["GMOE_DECODE_KERNEL"] = old


@pytest.fixture(params=list(DECODE_KERNELS))
def dkernel(request):
    """Runs the test once per persistent T=1 kernel (contexts created in the test)."""
    with decode_kernel(request.param):
        yield request.param


def launched(ctx, run):
    """gmoe_profile bucket names of the kernels that run() launched on ctx."""
    ctx.profile(True)
    run()
    prof = ctx.profile_read()
    ctx.profile(False)
    return set(prof)


def assert_decode_kernel(ran, kind):
    """The persistent T=1 kernel of `kind` ran, and the other one did not."""
    assert DECODE_KERNEL_NAMES[kind] in ran, ran
    assert not (set(DECODE_KERNEL_NAMES.values()) - {DECODE_KERNEL_NAMES[kind]}) & ran, ran


@pytest.fixture(scope="session")
def gpu_available():
    import gmoe
    try:
        return gmoe.device_count() > 0
    except OSError:
        return False


@pytest.fixture(autouse=True)
def _require_gpu_for_gpu_tests(request):
    if request.node.get_closest_marker("gpu") is not None:
        import gmoe
        n = 0
        try:
            n = gmoe.device_count()
        except OSError:
            pass
        if n == 0:
            pytest.fail("gpu test but no HIP device is visible")


@pytest.fixture(scope="session")
def glm_layer1():
    """GLM-4.7-Flash layer 1 weights (seed 0), as the golden fixtures used them."""
    import gmoe
    return gmoe.HostLayer(gmoe.GLM47_FLASH, seed=0, layer=1)


@pytest.fixture(scope="session")
def glm_layer1_zipf():
    import gmoe
    return gmoe.HostLayer(gmoe.GLM47_FLASH, seed=0, layer=1, bias_mode=gmoe.SYNTH_BIAS_ZIPF)
