"""Run ResKV and dense inference for each batch size in separate, sequential
processes, check that the reports are comparable, and write a summary.
``python -m reskv_amd.benchmarks.compare --model <dir> ...`` (the reference's
benchmarks/compare.py without its Mustafar method, which is out of scope)."""

import argparse
import json
import statistics
import subprocess
import sys
from pathlib import Path

from .common import check_run, declare_run, require_gpu, save_json

# report fields that must agree across the methods of one batch size
SHARED_FIELDS = ("model", "model_dtype", "batch_size", "input_length", "new_tokens", "seed", "input_ids_sha256",
                 "git_commit", "source_sha256", "gpu", "torch", "hip", "repeats", "warmup")
SUMMARY_FIELDS = ("prefill_ms", "decode_ms", "tpot_ms", "throughput_tps")


def validate_reports(reports):
    """Raise ValueError unless the reports describe the same inputs and environment,
    hold ``repeats`` records each, and every record decoded new_tokens - 1 steps with
    finite final logits."""
    base = reports[0]
    for rep in reports:
        mismatched = [f for f in SHARED_FIELDS if rep[f] != base[f]]
        if mismatched:
            raise ValueError(f"comparison mismatch in {mismatched[0]}")
        if len(rep["records"]) != rep["repeats"]:
            raise ValueError("unexpected record count")
        if any(r["decode_steps"] != rep["new_tokens"] - 1 or not r["finite_last_logits"] for r in rep["records"]):
            raise ValueError("decode step count does not match output length, or nonfinite logits")


def summary_row(report, path):
    """Median of each timing over the report's records, and the peak allocation."""
    row = {"method": report["method"], "batch_size": report["batch_size"], "result": str(path)}
    for name in SUMMARY_FIELDS:
        seen = [r[name] for r in report["records"] if r[name] is not None]
        row[name] = statistics.median(seen) if seen else None
    row["peak_allocated_bytes"] = max(r["peak_allocated_bytes"] for r in report["records"])
    return row


def child_command(args, method, batch_size, output):
    cmd = [sys.executable, "-m", "reskv_amd.benchmarks.inference", "--method", method, "--dtype", args.dtype,
           "--model", args.model, "--batch-size", str(batch_size), "--input-length", str(args.input_length),
           "--new-tokens", str(args.new_tokens), "--seed", str(args.seed), "--warmup", str(args.warmup),
           "--repeats", str(args.repeats), "--output", str(output)]
    if method == "reskv":
        cmd += ["--sparsity", str(args.sparsity), "--reskv-implementation", args.reskv_implementation]
    return cmd


def _run_one(args, method, batch_size):
    target = args.output / f"{method}-b{batch_size}.json"
    log = target.with_suffix(".log")
    target.unlink(missing_ok=True)
    print(f"Running {method}, batch={batch_size}; log: {log}", flush=True)
    with log.open("w", encoding="utf-8") as stream:
        subprocess.run(child_command(args, method, batch_size, target), check=True, stdout=stream,
                       stderr=subprocess.STDOUT)
    report = json.loads(target.read_text(encoding="utf-8"))
    if report["method"] != method:
        raise ValueError("result method does not match requested method")
    return report, target, log


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    declare_run(parser, many_batches=True)
    parser.add_argument("--methods", nargs="+", choices=["reskv", "dense"], default=["reskv", "dense"])
    parser.add_argument("--output", type=Path, default=Path("results/comparison"))
    args = parser.parse_args()
    check_run(parser, args)
    if args.dtype != "fp16" and "reskv" in args.methods:
        parser.error("comparisons including ResKV require --dtype fp16")
    if len(set(args.methods)) != len(args.methods) or len(set(args.batch_sizes)) != len(args.batch_sizes):
        parser.error("methods and batch sizes must not contain duplicates")
    require_gpu(parser)
    args.output.mkdir(parents=True, exist_ok=True)
    summary = {"runs": [], "errors": []}
    for batch_size in args.batch_sizes:
        reports, rows = [], []
        for method in args.methods:
            try:
                report, target, _ = _run_one(args, method, batch_size)
                reports.append(report)
                rows.append(summary_row(report, target))
            except (OSError, subprocess.CalledProcessError, ValueError, KeyError) as exc:
                log = args.output / f"{method}-b{batch_size}.log"
                summary["errors"].append({"method": method, "batch_size": batch_size, "error": str(exc),
                                          "log": str(log)})
        if not reports:
            continue
        try:
            validate_reports(reports)
            summary["runs"].extend(rows)
        except (ValueError, KeyError) as exc:
            summary["errors"].append({"batch_size": batch_size, "error": str(exc)})
    path = args.output / "summary.json"
    save_json(path, summary)
    print(f"Results: {path}")
    if summary["errors"]:
        raise SystemExit(1)


if __name__ == "__main__":
    main()
