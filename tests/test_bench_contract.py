"""The benchmark's contract with its driver: ``python bench.py`` prints exactly one JSON line on
stdout, with BASELINE.json's metric, whole-job ``value`` consistent with ``ms_per_step``, and the
roofline of the dominant kernel; ``--gpus N`` above 1 exits with a message (one GPU is measured).
The GPU case runs the script as the driver does, in a child process, with few steps."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
BENCH = REPO / "bench.py"


def _run(*args: str, timeout: float):
    return subprocess.run([sys.executable, str(BENCH), *args], cwd=REPO, capture_output=True, text=True,
                          timeout=timeout)


def test_more_than_one_gpu_is_refused_before_any_device_work():
    p = _run("--gpus", "2", timeout=120)
    assert p.returncode == 2
    assert p.stdout == ""
    assert "one GPU only" in p.stderr


@pytest.mark.gpu
def test_one_json_line_with_the_baseline_metric_and_a_consistent_roofline(cuda):
    p = _run("--steps", "3", "--warmup", "1", "--settle-ms", "20", "--no-cpu-baseline", timeout=170)
    assert p.returncode == 0, p.stderr[-2000:]
    lines = [ln for ln in p.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, p.stdout[-2000:]
    line = json.loads(lines[0])
    baseline = json.loads((REPO / "BASELINE.json").read_text())
    assert line["metric"] == baseline["metric"]
    for key in ("value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
                "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 3 and line["warmup"] == 1
    assert line["higher_is_better"] is True and line["unit"] == "TFLOPS"
    assert "workload" in line["config"] and "model" not in line["config"]
    # whole-job throughput of the timed steps: 2 * 4096^3 flop per step (within the rounding of both)
    flop = 2.0 * 4096 ** 3
    assert line["value"] == pytest.approx(flop / (line["ms_per_step"] * 1e-3) / 1e12, rel=2e-3)
    r = line["roofline"]
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["peak"] == pytest.approx(2516.6)
    assert r["frac"] == pytest.approx(r["achieved"] / r["peak"], abs=1e-4)
    assert r["achieved"] == pytest.approx(flop / (r["kernel_ms"] * 1e-3) / 1e12, rel=2e-3)
    assert 0 < r["frac"] < 1 and isinstance(r["traffic"], int) and r["traffic"] > 0
    # the GEMM kernel is part of each step, so it cannot take longer than the step
    assert r["kernel_ms"] < line["ms_per_step"]
    s = line["skinny_m1"]["roofline"]
    assert s["bound"] == "hbm" and s["unit"] == "GB/s" and 0 < s["frac"] < 1
    assert s["frac"] == pytest.approx(s["achieved"] / s["peak"], abs=1e-4)
