"""The drop-in builds: glm.c's own app, patched as INTEGRATION.md section 1 shows
(--backend hip, GLM_BACKEND=hip, the MoE hook at infer.c:1087, batched prefill at
infer.c:2178), compiles and links against libglm_hip.so in place of backend.c
(oracle/build_app.py), and with the CPU backend it writes exactly what the unpatched
reference app writes. Without a GPU, --backend hip ends as backend.c ends a failed
init (backend.c:76-82: a message and exit status 1)."""
import os

import pytest

import app_runner
import gmoe

pytestmark = pytest.mark.skipif(not app_runner.available(),
                                reason="glm.c's app not built (needs the reference sources)")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    return app_runner.write_model(tmp_path_factory.mktemp("app"), app_runner.small_spec())


def test_patched_app_with_cpu_backend_writes_what_glm_writes(model):
    args = ["-n", "12", "-i", app_runner.PROMPT, "-t", "0"]
    ref = app_runner.run("cpu", model, args)
    got = app_runner.run("hip", model, args + ["--backend", "cpu"])
    assert ref.returncode == 0, ref.stderr
    assert got.returncode == 0, got.stderr
    assert app_runner.generated(got.stdout) == app_runner.generated(ref.stdout)
    assert "backend=cpu" in got.stdout


def test_patched_app_bench_report_with_cpu_backend(model, tmp_path):
    rep = tmp_path / "report.json"
    r = app_runner.run("hip", model, ["-n", "6", "-i", "abc", "--bench-mode", "full", "--bench-report", str(rep),
                                      "--backend", "cpu"])
    assert r.returncode == 0, r.stderr
    j = app_runner.bench_report(rep)
    assert j["backend"] == "cpu"
    assert j["decode"]["tokens"] >= 1 and j["decode"]["p50_ms"] > 0


def test_metal_request_exits_as_backend_c_does(model):
    r = app_runner.run("hip", model, ["-n", "2", "-i", "abc", "--backend", "metal"])
    assert r.returncode == 1
    assert "[glm-metal] unavailable" in r.stderr


def test_hip_backend_without_a_device_exits_with_a_message(model):
    try:
        n = gmoe.device_count()
    except OSError:
        n = 0
    if n:
        pytest.skip("a HIP device is visible")
    for extra, env in ((["--backend", "hip"], None), ([], {"GLM_BACKEND": "hip"})):
        r = app_runner.run("hip", model, ["-n", "2", "-i", "abc"] + extra, env=env)
        assert r.returncode == 1, (extra, env, r.stdout, r.stderr)
        assert "[glm-hip] init failed" in r.stderr
        assert "backend=hip" in r.stdout


def test_patched_app_debug_lines_with_cpu_backend(model):
    args = ["-n", "3", "-i", "abcd", "-t", "0", "--debug"]
    ref = app_runner.run("cpu", model, args)
    got = app_runner.run("hip", model, args + ["--backend", "cpu"])
    assert ref.returncode == 0 and got.returncode == 0
    pick = lambda e: [ln for ln in e.splitlines() if ln.startswith("[glm-layer-sum]")]  # noqa: E731
    assert pick(got.stderr) == pick(ref.stderr) and len(pick(ref.stderr)) > 25
