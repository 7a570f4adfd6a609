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


def test_counter_records_cover_the_bench_workloads():
    """Every workload the line reports a roofline for has a committed counter
    record: config 2 at both sparsities (B = 32) and config 3 at INT4 / INT2."""
    sys.path.insert(0, str(ROOT))
    import bench

    for key in ((32, 8192, 0.5, "unstructured", 16), (32, 8192, 0.75, "structured", 16),
                (8, 16384, 0.5, "unstructured", 4), (8, 16384, 0.5, "unstructured", 2)):
        rec = bench.counter_record(*key)
        assert rec is not None, key
        assert rec["fetch_bytes"] > 0 and rec["units"] == key[0] * 8 * key[1]
        traffic, source = bench.measured_traffic(rec, rec["splits"])
        assert traffic == rec["fetch_bytes"] + rec["write_bytes"]
        assert source["measured_at_splits"] == source["this_run_splits"]
    assert bench.counter_record(32, 8192, 0.5, "unstructured", 4) is None
    assert bench.measured_traffic(None, 2) == (None, None) and bench.issue_ceiling(None, 1, 0.1) is None


def test_issue_ceiling_arithmetic():
    """A kernel issuing V VALU instructions per unit on 1024 SIMDs at f GHz
    spends 4 V / (1024 f) ns per unit; the ceiling is the bandwidth at that rate."""
    sys.path.insert(0, str(ROOT))
    import bench

    rec = {"valu_per_unit": 20.0, "mfma_per_unit": 2.0, "units": 1 << 20, "clock_ghz": 2.0}
    nbytes = 100 * (1 << 20)  # 100 B per unit
    c = bench.issue_ceiling(rec, nbytes, 0.25)
    seconds = (1 << 20) * 80 / (1024 * 2.0e9)
    assert abs(c["valu_issue_ceiling_frac"] - nbytes / seconds / 8.0e12) < 1e-12
    assert abs(c["valu_issue_ceiling_frac"] - 0.32) < 1e-12  # 100 B per 80 / (1024 * 2 GHz) s = 2.56 TB/s
    assert abs(c["frac_of_ceiling"] - 0.25 / 0.32) < 1e-12
