"""bench.py's command-line contract that needs no GPU: a multi-GPU request
exits at once with a message (this build measures one GPU), and the
roofline traffic it reports comes from the committed rocprofv3 summary."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + args,
                          capture_output=True, text=True, timeout=120, env=env)


def test_multi_gpu_request_exits_with_message():
    res = run_bench(["--gpus", "2"])
    assert res.returncode == 2
    assert "one GPU" in res.stderr and res.stdout == ""


def test_world_size_above_one_exits_with_message():
    res = run_bench([], {"WORLD_SIZE": "4"})
    assert res.returncode == 2
    assert "WORLD_SIZE 4" in res.stderr


def test_roofline_traffic_from_committed_summary():
    sys.path.insert(0, ROOT)
    import bench

    with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
        data = json.load(f)
    k = data["kernels"]["forge_gemm_nn_64x128x32_x8"]
    want = round(k["fetch_kib"] * 1024 * data["fetch_factor"] +
                 k["write_kib"] * 1024 * data["write_factor"])
    assert bench.load_traffic("forge_gemm_nn_64x128x32_x8") == want
    # The counters cover at least the algorithmic bytes of the product.
    assert want >= k["algorithmic_read_bytes"] + k["algorithmic_write_bytes"]
    assert bench.load_traffic("no_such_kernel") is None
