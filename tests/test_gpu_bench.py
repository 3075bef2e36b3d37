"""The bench line the round's driver reads: one JSON line on stdout with the contract's keys.

Runs `bench.py --steps 5 --warmup 2 --no-side` in a child process (config 2's decode step, the
roofline of the v1 call and the CPU baseline) and checks the line's keys, types and the
relations between its figures (value from the step time and bytes, roofline fraction from
achieved / peak), so that a change to the bench cannot silently break what the driver parses.
"""
from __future__ import annotations

import json
import math
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_line_contract():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--steps", "5", "--warmup", "2", "--no-side"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, r.stdout[-2000:]
    d = json.loads(lines[0])
    for key, typ in (("metric", str), ("value", float), ("unit", str), ("n_gpus", int), ("steps", int),
                     ("warmup", int), ("ms_per_step", float), ("higher_is_better", bool), ("scaling", str),
                     ("dtype", str), ("data", str), ("config", dict), ("roofline", dict), ("cpu_baseline", dict)):
        assert isinstance(d[key], typ), (key, d.get(key))
    assert "vs_baseline" in d and d["vs_baseline"] is None
    assert d["n_gpus"] == 1 and d["steps"] == 5 and d["warmup"] == 2 and d["settle_ms"] > 0
    assert d["unit"] == "GB/s" and d["higher_is_better"] is True and d["scaling"] == "weak" and d["dtype"] == "bf16"
    assert d["config"]["workload"].startswith("config2")
    # value = the step's algorithmic bytes / step time
    step_bytes = d["value"] * 1e9 * d["ms_per_step"] * 1e-3
    assert 5.8e8 < step_bytes < 6.0e8, step_bytes
    rf = d["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert math.isclose(rf["frac"], rf["achieved"] / rf["peak"], rel_tol=1e-3)
    assert math.isclose(rf["achieved"], rf["algorithmic_bytes"] / (rf["us_per_launch"] * 1e-6) / 1e9, rel_tol=1e-2)
    assert 0.3 < rf["frac"] < 1.0
    assert rf["traffic"] is None or rf["traffic"] > rf["algorithmic_bytes"] * 0.99
    cb = d["cpu_baseline"]
    assert cb["value"] > 0 and cb["cores"] >= 1 and cb["kind"] in ("port", "reference") and cb["sample"]
