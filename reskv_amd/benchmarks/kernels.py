"""Event-timed sweep of the ``compress`` and ``attention`` APIs over batch
sizes and sparsities at one context length (the reference's
benchmarks/kernels.py command line and record fields).  ``python -m
reskv_amd.benchmarks.kernels [--batch-sizes 1 16] [--seq-len 8192] ...``

Inputs follow the reference's recipe (seed 42: K, V = 0.5 N(0,1), centres
0.1 N(0,1), random ids, one 0.5 N(0,1) query per head, 8 KV and 32 query
heads), compressed with that external clustering so the timing excludes
K-means.  Each record carries two checks: ``split_invariance_max_abs``, the
largest difference between the automatic split count and 16 splits (the
split-K merge must not change the result), and, when the caller passes a
``checker`` (the test suite passes a float32 reconstruction), the
``max_abs_error`` against it.
"""

import argparse
import json
from pathlib import Path

import torch

from .. import ResKVKernelConfig, attention, compress
from .common import median_event_ms, provenance, require_gpu, save_json

KV_HEADS, QUERY_HEADS, CENTRES = 8, 32, 32


def _inputs(batch, seq_len):
    torch.manual_seed(42)
    shape = (batch, KV_HEADS, seq_len, 128)
    dev = "cuda"
    kv = [torch.randn(shape, device=dev, dtype=torch.float16) * 0.5 for _ in range(2)]
    centres = [torch.randn(batch, KV_HEADS, CENTRES, 128, device=dev, dtype=torch.float16) * 0.1 for _ in range(2)]
    ids = [torch.randint(CENTRES, shape[:3], device=dev, dtype=torch.int32) for _ in range(2)]
    q = torch.randn(batch, QUERY_HEADS, 1, 128, device=dev, dtype=torch.float16) * 0.5
    return kv, ((centres[0], ids[0]), (centres[1], ids[1])), q


def sweep(batch_sizes, seq_len, sparsities, implementation="default", checker=None):
    """Yield one record per (batch size, sparsity)."""
    layout = "unstructured" if implementation == "unstructure" else "auto"
    for batch in batch_sizes:
        for sparsity in sparsities:
            cfg = ResKVKernelConfig(sparsity=sparsity, layout=layout)
            (k, v), clustering, q = _inputs(batch, seq_len)
            make = lambda: compress(k, v, cfg, clustering=clustering)  # noqa: E731
            cache = make()
            decode = lambda: attention(q, cache, position=seq_len)  # noqa: E731
            out = decode().float()
            other = attention(q, cache, position=seq_len, splits=16).float()
            record = {
                "kernel_config": cfg.to_dict(),
                "kernel_plan": cache.key.plan.to_dict(),
                "batch_size": batch,
                "seq_len": seq_len,
                "decode_ms": median_event_ms(decode),
                "compression_ms": median_event_ms(make),
                "split_invariance_max_abs": (out - other).abs().max().item(),
                "max_abs_error": None,
                "cache_bytes": cache.nbytes,
            }
            if checker is not None:
                record["max_abs_error"] = (out - checker(q, cache, position=seq_len).float()).abs().max().item()
            yield record
            del k, v, clustering, q, cache, out, other
            torch.cuda.empty_cache()


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--batch-sizes", type=int, nargs="+", default=[1, 16])
    parser.add_argument("--seq-len", type=int, default=8192)
    parser.add_argument("--sparsities", type=float, nargs="+", choices=[0.5, 0.75], default=[0.5, 0.75])
    parser.add_argument("--reskv-implementation", choices=["default", "unstructure"], default="default",
                        help="ResKV implementation; default selects automatically for the sparsity and batch size")
    parser.add_argument("--output", type=Path, default=Path("results/kernels.json"))
    args = parser.parse_args()
    if args.seq_len < 1 or min(args.batch_sizes) < 1:
        parser.error("sequence length and batch sizes must be positive")
    require_gpu(parser)
    records = []
    for rec in sweep(args.batch_sizes, args.seq_len, args.sparsities, args.reskv_implementation):
        if rec["split_invariance_max_abs"] > 2e-3:
            raise RuntimeError(f"split-count invariance violated: {rec}")
        print(json.dumps(rec), flush=True)
        records.append(rec)
    save_json(args.output, {**provenance(), "records": records})


if __name__ == "__main__":
    main()
