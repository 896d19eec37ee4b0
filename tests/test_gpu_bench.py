"""bench.py on the GPU, as the round-end driver runs it: one JSON line on
stdout with the contract's keys, the roofline and CPU-baseline objects, and
the single-workload mode used for profiling."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args, timeout=240):
    print("bench.py", *args, flush=True)
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                         capture_output=True, text=True, timeout=timeout)
    assert out.returncode == 0, out.stderr[-2000:]
    lines = [ln for ln in out.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, out.stdout
    return json.loads(lines[0])


def test_headline_line_keeps_the_contract():
    d = _run("--no-suite", "--steps", "3", "--warmup", "2")
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 2
    assert d["value"] > 0 and d["ms_per_step"] > 0 and d["higher_is_better"] is True
    assert d["vs_baseline"] is None and d["dtype"] == "fp32"
    assert d["config"]["M"] == d["config"]["N"] == d["config"]["K"] == 4096
    # value is the whole loop's GFLOP/s: 2 * 4096^3 per step over ms_per_step
    assert abs(d["value"] - 2 * 4096 ** 3 / (d["ms_per_step"] * 1e-3) / 1e9) / d["value"] < 0.01
    r = d["roofline"]
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["peak"] == 157.3
    assert 0 < r["frac"] < 1 and abs(r["frac"] - r["achieved"] / r["peak"]) < 1e-3
    assert r["traffic"] > 0 and r["traffic_source"]["kernels"]
    assert 0 < r["mfma_busy"] <= 1 and r["mfma_busy_source"]["kernels"]
    c = d["cpu_baseline"]
    assert c["value"] > 0 and c["cores"] == 1 and c["kind"] == "port" and c["sample"]


def test_single_workload_mode():
    d = _run("--workload", "skinny", "--steps", "5", "--warmup", "2")
    assert d["workload"] == "skinny"
    assert d["ms"] > 0 and d["bytes"] == 4.0 * (16 * 4096 + 4096 * 4096 + 16 * 4096)
    d = _run("--workload", "gemm1024", "--steps", "5", "--warmup", "2")
    assert d["workload"] == "gemm1024" and d["ms"] > 0 and d["value"] > 0
