"""bench.py's output contract: one JSON line with the metric, the whole-job
value, roofline and the side figures.  The CPU case checks that more than one
GPU is refused with a message; the GPU case runs a small workload end to end
(200k points of the 1M workload's mixture, the query set repeated 3 times per
step) and checks every key the driver and the design notes read."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _run(*args, timeout=600):
    r = subprocess.run([sys.executable, "-u", str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                       timeout=timeout, cwd=ROOT)
    lines = [ln for ln in r.stdout.strip().splitlines() if ln.startswith("{")]
    return r.returncode, (json.loads(lines[-1]) if lines else None), r.stderr


def test_more_than_one_gpu_is_refused():
    rc, out, _ = _run("--gpus", "2", timeout=120)
    assert rc == 2
    assert out["n_gpus"] == 2 and "one GPU" in out["error"]


@pytest.mark.gpu
def test_small_bench_line():
    from quiver import _lib

    if _lib.device_count() == 0:
        pytest.skip("no GPU")
    print("[gpu] bench.py small workload, repeat 3", flush=True)
    rc, out, err = _run("--workload", "small-1M-u8", "--n", "200000", "--steps", "2", "--warmup", "1",
                        "--repeat", "3", "--no-cpu", "--no-adc", "--latency-batches", "1",
                        "--open-loop-batches", "")
    assert rc == 0, err[-2000:]
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "host_buffers", "single_batch"):
        assert key in out, key
    assert out["n_gpus"] == 1 and out["steps"] == 2 and out["dtype"] == "u8" and out["value"] > 0
    c = out["config"]
    assert c["repeat"] == 3 and c["queries_per_step"] == 30000 and c["repeats_identical"] is True
    assert out["host_buffers"]["same_results"] is True
    assert out["single_batch"]["device_resident"]["same_results"] is True
    assert out["single_batch"]["host_buffers"]["same_results"] is True
    r = out["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in r, key
    assert r["queries_per_launch"] == 30000 and 0 < r["frac"] < 1
    assert abs(r["frac"] - r["achieved"] / r["peak"]) < 1e-3
    assert out["latency_mode"] and out["latency_mode"][0]["batch"] == 1
