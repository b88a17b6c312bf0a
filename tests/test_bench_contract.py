"""CPU checks of bench.py's contract (no GPU): a multi-GPU request exits with
a message instead of measuring, and the two CPU legs of the JSON line carry
the fields the line reports (value, unit, cores, kind, sample)."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       cwd=ROOT, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""          # no JSON line for an unmeasured configuration


def test_cpu_legs_report_the_json_fields():
    ref = bench.cpu_baseline(1, 0.3)
    port = bench.cpu_port(1, 0.3)
    for leg, kind in ((ref, "reference"), (port, "port")):
        assert set(leg) >= {"value", "unit", "cores", "kind", "sample"}
        assert leg["kind"] == kind and leg["unit"] == "GB/s"
        assert leg["value"] > 0 and leg["cores"] >= 1 and "steps" in leg["sample"]
