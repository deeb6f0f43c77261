"""bench.py's output line on the device: one JSON line on stdout with every
field the benchmark contract names, the roofline object of the decode kernel
(algorithmic bytes over the measured launch time, against the 8 TB/s HBM
peak) and the value consistent with the bytes and the time per step. A short
run (2 timed steps, decode only, no CPU baseline); the figures themselves are
measured by the full run, not here."""
import json
import os
import subprocess
import sys

import pytest

import bench

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_json_line():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--steps", "2", "--warmup", "1",
                        "--only", "decode", "--no-cpu"], capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [x for x in r.stdout.splitlines() if x.strip()]
    assert len(lines) == 1, r.stdout
    out = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline"):
        assert key in out, key
    assert out["n_gpus"] == 1 and out["steps"] == 2 and out["warmup"] == 1
    assert out["unit"] == "GB/s" and out["higher_is_better"] is True and out["vs_baseline"] is None
    assert "workload" in out["config"]
    nbytes = bench.decode_bytes(24, 4096, 14, 2, 64, 4)
    assert out["value"] == pytest.approx(nbytes / (out["ms_per_step"] * 1e-3) / 1e9, rel=1e-3)
    roof = out["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in roof, key
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"], abs=1e-4)
    assert 0.0 < roof["frac"] < 1.0
