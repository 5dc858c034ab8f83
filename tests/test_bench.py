"""The output contract of bench.py: one JSON line with the headline fields,
`roofline`, `cpu_baseline` and the measured ceilings; one GPU only."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args, timeout=300):
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT, capture_output=True,
                       text=True, timeout=timeout)
    lines = [line for line in p.stdout.splitlines() if line.startswith("{")]
    return p.returncode, lines, p.stderr


def test_more_than_one_gpu_is_refused():
    rc, lines, _ = run_bench("--gpus", "2", timeout=120)
    assert rc == 2
    assert len(lines) == 1
    out = json.loads(lines[0])
    assert out["n_gpus"] == 2 and "one GPU" in out["error"]


@pytest.mark.gpu
def test_headline_line(hip):
    rc, lines, err = run_bench("--steps", "3", "--warmup", "1", "--no-extra", "--cpu-seconds", "1")
    assert rc == 0, err[-2000:]
    assert len(lines) == 1
    out = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "measured_peaks"):
        assert key in out, key
    assert out["n_gpus"] == 1 and out["steps"] == 3 and out["warmup"] == 1
    assert out["unit"] == "GB/s" and out["higher_is_better"] is True and out["dtype"] == "f32"
    assert out["vs_baseline"] is None and out["data"] == "synthetic"
    assert "C2" in out["config"]["workload"]
    # value = 10 launches of 64 MiB (plus outputs) per step over the step time
    step_bytes = 10 * 4096 * 4096 * 4
    assert out["value"] == pytest.approx(step_bytes / (out["ms_per_step"] * 1e-3) / 1e9, rel=0.01)
    assert 500.0 < out["value"] < 8000.0
    r = out["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in r, key
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert r["frac"] == pytest.approx(r["achieved"] / r["peak"], abs=1e-3)
    c = out["cpu_baseline"]
    assert c["kind"] == "port" and c["cores"] == 1 and c["unit"] == "GB/s" and c["value"] > 0 and c["sample"]
    m = out["measured_peaks"]
    assert 1000.0 < m["read_GBps"] < 8000.0 and 1000.0 < m["copy_GBps"] < 8000.0
