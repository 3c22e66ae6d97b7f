"""A persistent decode launch whose dependency waits give up must be reported, and must not
overwrite the caller's activations.

The host forces the condition: GMOE_SPIN_LIMIT=0 makes every wait of the persistent kernel
give up at its first poll that finds the producer not done. Every block still exits
normally (a failed wait returns from the kernel), so no GPU work is left hanging."""
import numpy as np
import pytest

import gmoe

pytestmark = pytest.mark.gpu

SMALL = gmoe.Shape(dim=256, moe_ffn_dim=256, n_routed_experts=16, n_experts_used=4)


@pytest.fixture
def starved_ctx(monkeypatch, dkernel):
    monkeypatch.setenv("GMOE_SPIN_LIMIT", "0")
    ctx = gmoe.Context(SMALL, n_layers=3, max_tokens=1)
    monkeypatch.delenv("GMOE_SPIN_LIMIT")
    for l in (1, 2):
        ctx.upload(l, gmoe.HostLayer(SMALL, seed=3, layer=l))
    yield ctx
    ctx.close()


def test_host_forward_reports_and_leaves_x_untouched(starved_ctx):
    x = gmoe.activations(3, 0, 1, SMALL.D)
    before = x.copy()
    print("[case] forced timeout through gmoe_forward_host (x_in aliases x_out)", flush=True)
    lib = starved_ctx.lib
    rc = lib.gmoe_forward_host(starved_ctx.h, 1, 1, gmoe.ptr(x), gmoe.ptr(x), 0, None)
    assert rc == -2, f"expected GMOE_ERR_HIP, got {rc}"
    assert "timed out" in gmoe.last_error()
    assert np.array_equal(x.view(np.uint32), before.view(np.uint32)), "x was overwritten by a failed launch"


def test_device_forward_reports_on_the_next_call(starved_ctx):
    x = gmoe.activations(3, 1, 1, SMALL.D)
    d_in = gmoe.DeviceArray.from_numpy(x)
    d_out = gmoe.DeviceArray(x.nbytes)
    print("[case] forced timeout through gmoe_forward_layers", flush=True)
    lib = starved_ctx.lib
    rc = lib.gmoe_forward_layers(starved_ctx.h, 1, 2, 1, d_in.ptr, d_out.ptr, 0, None)
    assert rc == 0  # asynchronous: the launch itself is accepted
    gmoe.hip_check(gmoe.hip().hipDeviceSynchronize(), "sync")
    rc = lib.gmoe_forward_layers(starved_ctx.h, 1, 2, 1, d_in.ptr, d_out.ptr, 0, None)
    assert rc == -2, "the failed launch before was not reported"
    assert "timed out" in gmoe.last_error()


def test_normal_context_after_a_failed_one(dkernel):
    """The failure is per context: a context with the default limit computes normally."""
    ctx = gmoe.Context(SMALL, n_layers=2, max_tokens=1)
    try:
        ctx.upload(1, gmoe.HostLayer(SMALL, seed=3, layer=1))
        x = gmoe.activations(3, 2, 1, SMALL.D)
        print("[case] normal launch after the forced timeouts", flush=True)
        got, st = gmoe.forward_host(ctx, 1, x)
        assert np.all(np.isfinite(got))
    finally:
        ctx.close()
