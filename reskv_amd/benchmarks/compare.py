"""Run ResKV and dense inference benchmarks in separate sequential processes and
check that their reports are comparable (benchmarks/compare.py of the reference;
the Mustafar baseline is not part of this build).  Run as
``python -m reskv_amd.benchmarks.compare``."""

import argparse
import json
import statistics
import subprocess
import sys
from pathlib import Path

from .._io import write_json
from .timing import add_arguments, add_model_arguments, validate_arguments, validate_gpu

_SAME = ("model", "model_dtype", "batch_size", "input_length", "new_tokens", "seed", "input_ids_sha256",
         "git_commit", "source_sha256", "gpu", "torch", "hip", "repeats", "warmup")


def validate_reports(reports):
    """Reject comparisons whose runs differ in inputs, environment or decode counts."""
    first = reports[0]
    for report in reports:
        for field in _SAME:
            if report[field] != first[field]:
                raise ValueError(f"comparison mismatch in {field}")
        if len(report["records"]) != report["repeats"]:
            raise ValueError("unexpected record count")
        for record in report["records"]:
            if record["decode_steps"] != report["new_tokens"] - 1 or not record["finite_last_logits"]:
                raise ValueError("decode step count does not match output length, or nonfinite logits")


def summarize(report, path):
    records = report["records"]
    row = {"method": report["method"], "batch_size": report["batch_size"], "result": str(path)}
    for name in ("prefill_ms", "decode_ms", "tpot_ms", "throughput_tps"):
        values = [record[name] for record in records if record[name] is not None]
        row[name] = statistics.median(values) if values else None
    row["peak_allocated_bytes"] = max(record["peak_allocated_bytes"] for record in records)
    return row


def command_for(args, method, batch_size, output):
    command = [sys.executable, "-m", "reskv_amd.benchmarks.inference", "--method", method, "--dtype", args.dtype,
               "--model", args.model, "--batch-size", str(batch_size), "--input-length", str(args.input_length),
               "--new-tokens", str(args.new_tokens), "--seed", str(args.seed), "--warmup", str(args.warmup),
               "--repeats", str(args.repeats), "--output", str(output)]
    if method == "reskv":
        command += ["--sparsity", str(args.sparsity), "--reskv-implementation", args.reskv_implementation]
    return command


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    add_arguments(parser, batch_sizes=True)
    parser.add_argument("--methods", nargs="+", choices=["reskv", "dense"], default=["reskv", "dense"])
    add_model_arguments(parser)
    parser.add_argument("--output", type=Path, default=Path("results/comparison"))
    args = parser.parse_args()
    validate_arguments(parser, args)
    if args.dtype != "fp16" and "reskv" in args.methods:
        parser.error("comparisons including ResKV require --dtype fp16")
    if len(set(args.methods)) != len(args.methods) or len(set(args.batch_sizes)) != len(args.batch_sizes):
        parser.error("methods and batch sizes must not contain duplicates")
    validate_gpu(parser)
    args.output.mkdir(parents=True, exist_ok=True)
    summary = {"runs": [], "errors": []}
    for batch_size in args.batch_sizes:
        reports, rows = [], []
        for method in args.methods:
            target = args.output / f"{method}-b{batch_size}.json"
            log = target.with_suffix(".log")
            target.unlink(missing_ok=True)
            print(f"Running {method}, batch={batch_size}; log: {log}", flush=True)
            try:
                with log.open("w", encoding="utf-8") as stream:
                    subprocess.run(command_for(args, method, batch_size, target), check=True, stdout=stream,
                                   stderr=subprocess.STDOUT)
                report = json.loads(target.read_text(encoding="utf-8"))
                if report["method"] != method:
                    raise ValueError("result method does not match requested method")
                reports.append(report)
                rows.append(summarize(report, target))
            except (OSError, subprocess.CalledProcessError, ValueError, KeyError) as exc:
                summary["errors"].append({"method": method, "batch_size": batch_size, "error": str(exc),
                                          "log": str(log)})
        if reports:
            try:
                validate_reports(reports)
                summary["runs"].extend(rows)
            except (ValueError, KeyError) as exc:
                summary["errors"].append({"batch_size": batch_size, "error": str(exc)})
    summary_path = args.output / "summary.json"
    write_json(summary_path, summary)
    print(f"Results: {summary_path}")
    if summary["errors"]:
        raise SystemExit(1)


if __name__ == "__main__":
    main()
