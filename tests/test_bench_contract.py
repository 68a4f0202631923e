"""bench.py's contract, checked without a GPU: every workload has a runner,
the default run's extra workloads exist, a multi-GPU request is refused
before anything touches a device, and the committed counter figures that the
bench lines carry as `roofline.traffic` are readable."""
import os
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_every_workload_has_a_runner():
    for name, w in bench.WORKLOADS.items():
        assert w.get("kind", "layer") in bench.RUNNERS, name
        assert w.get("desc"), name


def test_default_extra_workloads_exist():
    names = [n for n, _ in bench.EXTRA_WORKLOADS]
    assert len(names) == len(set(names))
    for n, steps in bench.EXTRA_WORKLOADS:
        assert n in bench.WORKLOADS and n != "c2" and steps >= 1
        assert bench.WORKLOADS[n].get("kind", "layer") not in ("gather", "stream", "launch")


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}),
                                      ([], {"WORLD_SIZE": "2"})])
def test_multi_gpu_request_refused(args, env):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                       timeout=120, env={**os.environ, **env})
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr
    assert r.stdout == ""


@pytest.mark.parametrize("profile,key", [
    ("moe_layer_c2_traffic.md", "traffic_bytes_per_call"),
    ("moe_layer_c3_traffic.md", "traffic_bytes_per_call"),
    ("dense_gemv_c1_traffic.md", "traffic_bytes_per_call"),
    ("mtp_verify_c4_traffic.md", "traffic_bytes_per_call"),
    ("mtp_verify_c4capped_traffic.md", "traffic_bytes_per_call"),
    ("dense_prefill_c5_traffic.md", "traffic_bytes_per_step"),
])
def test_committed_traffic_figures_read(profile, key):
    v = bench.measured_traffic(profile, key)
    assert isinstance(v, (int, float)) and v > 0, (profile, key, v)
