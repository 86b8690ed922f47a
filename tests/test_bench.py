"""bench.py's host-side pieces, on the CPU: the rocprofv3 counter parsing behind `roofline.traffic`, the
committed traffic table it falls back to, and the one-GPU guard of the driver's --gpus N contract."""
import importlib.util
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
bench = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(bench)


def _rows(entries):
    return [{"Dispatch_Id": str(i + 1), "Kernel_Name": n, "Counter_Value": str(v)} for i, (n, v) in enumerate(entries)]


def test_counter_bytes_calibrates_on_the_copies_and_drops_the_replays():
    # forwards: two Wqkv launches (100, 200 units) and one Wi launch (50); then 51 replays of Wqkv (9999 each,
    # left out); then three 256 MiB copies reading 131072 units each -> 2048 bytes per unit.
    qkv = "void (anonymous namespace)::gemm_ws_kernel<1>(GemmArgs, int, int, int)"
    wi = "void (anonymous namespace)::gemm_ws_kernel<2>(GemmArgs, int, int, int)"
    entries = [("__amd_rocclr_copyBuffer", 4.0), (qkv, 100), (wi, 50), ("layer_norm_kernel<12>", 7), (qkv, 200)]
    entries += [(qkv, 9999)] * 51 + [("__amd_rocclr_copyBuffer", 131072)] * 3
    got = bench.counter_bytes(_rows(entries))
    assert got == {"gemm_qkv_rope": 150 * 2048.0, "gemm_wi_geglu": 50 * 2048.0}


def test_counter_bytes_needs_the_copy_calibration():
    qkv = "gemm_ws_kernel<1>"
    assert bench.counter_bytes(_rows([(qkv, 1)] * 60)) is None
    assert bench.counter_bytes(_rows([(qkv, 1)] * 60 + [("__amd_rocclr_copyBuffer", 0)] * 3)) is None


def test_committed_traffic_reads_the_profile_table():
    traffic, commit = bench.committed_traffic("gemm_qkv_rope", "config1")
    assert isinstance(traffic, int) and traffic > 61_796_352  # at least the algorithmic bytes
    with open(os.path.join(ROOT, "profiles", "traffic.md")) as f:
        assert f"csrc commit: {commit}" in f.read()
    assert bench.committed_traffic("gemm_qkv_rope", "no-such-workload")[0] is None


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=60, env={**os.environ, "WORLD_SIZE": "1"})
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["skipped"] and line["n_gpus"] == 2 and "one GPU" in line["error"]
