"""bench.py's command-line contract that needs no GPU: more than one GPU is
refused with a message, and the JSON line's metric names the headline."""

import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused_with_a_message():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == 2
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_metric_is_the_baseline_metric():
    sys.path.insert(0, str(ROOT))
    import bench

    baseline = json.loads((ROOT / "BASELINE.json").read_text())
    assert bench.METRIC == baseline["metric"]
