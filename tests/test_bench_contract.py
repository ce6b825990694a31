"""bench.py keeps the driver's contract: one JSON line with the metric, the
step timing, the roofline and the CPU baseline; more than one GPU is refused
with a message."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KEYS = ["metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
        "scaling", "vs_baseline", "dtype", "data", "config", "roofline"]
ROOFLINE = ["bound", "achieved", "peak", "unit", "frac", "traffic"]


def _bench(*args, timeout=240):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=timeout)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2", timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_every_config_is_described():
    """Each --config choice has a workload name, a kernel name and (except
    the einsum caller) a workloads.py configuration, and either a CPU sample
    size or a stated reason for having no CPU baseline."""
    sys.path.insert(0, ROOT)
    import bench
    import workloads

    for name in ("P", "C1", "C2", "C3", "C4", "C5", "M1", "F1", "F2"):
        assert name in bench.WORKLOAD_NAMES and name in bench.KERNEL_NAMES, name
        assert name in workloads.CONFIGS, name
        assert name == "P" or name in bench.CPU_ROWS or name in bench.NO_CPU_BASELINE, name
        if workloads.CONFIGS[name]["dtype"] == "f64":
            assert bench.WORKLOAD_NAMES[name].startswith(f"{name}: MaxPlus f64")


@pytest.mark.gpu
@pytest.mark.parametrize("args", [("--config", "P", "--cpu-rows", "64"),
                                  ("--config", "C1"),
                                  ("--config", "M1"), ("--config", "E1"), ("--config", "F2")],
                         ids=["P", "C1", "M1", "E1", "F2"])
def test_json_line(args):
    print(f"[case] bench.py {' '.join(args)}", flush=True)
    r = _bench(*args, "--steps", "2", "--warmup", "1")
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, r.stdout
    out = json.loads(lines[0])
    for key in KEYS:
        assert key in out, key
    assert out["n_gpus"] == 1 and out["steps"] == 2 and out["warmup"] == 1
    assert out["higher_is_better"] is True and out["value"] > 0 and out["ms_per_step"] > 0
    assert "workload" in out["config"]
    for key in ROOFLINE:
        assert key in out["roofline"], key
    roof = out["roofline"]
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    if args[1] == "M1":  # short K: HBM-bound, GB/s against 8 TB/s
        assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
        assert out["argmax_consistency_check"] is True
    if args[1] in ("P", "C1", "M1"):
        base = out["cpu_baseline"]
        assert base["value"] > 0 and base["cores"] == 1 and base["kind"] in ("port", "reference")
        assert "argmax" in base["sample"]
        assert out["argmax_consistency_check"] is True
    if args[1] == "F2":  # f64: against the FP64 vector peak; the reference's AVX2 f64 path
        assert roof["unit"] == "TFLOP/s" and roof["peak"] == 78.6 and out["dtype"] == "f64"
        base = out["cpu_baseline"]
        assert base["value"] > 0 and base["cores"] == 1 and base["kind"] == "port"
        assert "F64_AVX2" in base["sample"]
    if args[1] == "C1":  # the reference's value-only CPU path on the same product
        base = out["cpu_baseline_value_only"]
        assert base["value"] > 0 and base["cores"] == 1 and "AVX2" in base["sample"]
