"""Decode-attention benchmark over the compressed KV cache on one MI355X.

Workload (Llama-3.1-8B layer shape): 32 query heads,
8 KV heads, head_dim 128, RoPE theta 500000, compressed context T = 8192,
synthetic KV following reskv benchmarks/kernels.py:57-65 (k, v ~ 0.5 N(0,1),
centroids ~ 0.1 N(0,1), random cluster ids, seed 42).  One *step* is one
decode step of a 32-layer model: 32 fused decode-attention calls, each on its
own layer cache (32 distinct caches, so the 256 MB Infinity Cache cannot hold
the working set).  ``value`` = batch * steps / elapsed (tokens/s).

The JSON line also carries the roofline of the decode attention (algorithmic
compressed bytes per call / measured time per call vs 8 TB/s) and a CPU
baseline: the numpy oracle (reconstruct + float64 attention) on a bounded
sample, timed on this host.

``--sweep`` additionally measures every batch size and sparsity of config 2
plus the dense fp16 baseline and prints one JSON line per point.
"""

import argparse
import json
import os
import sys
import time

HBM_PEAK = 8.0e12  # bytes/s, MI355X HBM3E
METRIC = "decode tok/s, Llama-3.1-8B-shape 8K ctx bs1-32; attn µs/step + % HBM peak"
LAYERS = 32
HQ, HK, D, T = 32, 8, 128, 8192


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--batch", type=int, default=32)
    p.add_argument("--sparsity", type=float, default=0.5)
    p.add_argument("--layout", default="auto")
    p.add_argument("--seq-len", type=int, default=T)
    p.add_argument("--layers", type=int, default=LAYERS)
    p.add_argument("--sweep", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    return p.parse_args()


def algorithmic_bytes(plan, b, t, nc_k, nc_v):
    """Compressed bytes one decode call must read (+ q read, out write)."""
    if plan is None:  # dense fp16
        per_tok = 2 * D * 2
        cent = 0
    else:
        if plan.bits == 16:
            payload = 2 * plan.nnz
            meta = 16
            scale = 0
        elif plan.layout == "structured":
            payload, meta, scale = 16, 8, 2
        else:
            payload, meta, scale = 4 * 4 * plan.bits, 0, 2
        per_tok = 2 * (1 + payload + meta + scale)
        cent = (nc_k + nc_v) * D * 2
    return b * HK * (t * per_tok + cent) + 2 * b * HQ * D * 2


def build_caches(torch, b, t, sparsity, layout, layers, device):
    from reskv_amd import ResKVKernelConfig, compress

    cfg = ResKVKernelConfig(sparsity=sparsity, layout=layout)
    torch.manual_seed(42)
    shape = (b, HK, t, D)
    k = torch.randn(shape, device=device, dtype=torch.float16) * 0.5
    v = torch.randn_like(k) * 0.5
    kc = torch.randn(b, HK, 32, D, device=device, dtype=torch.float16) * 0.1
    vc = torch.randn_like(kc) * 0.1
    ki = torch.randint(32, (b, HK, t), device=device, dtype=torch.int32)
    vi = torch.randint(32, (b, HK, t), device=device, dtype=torch.int32)
    base = compress(k, v, cfg, clustering=((kc, ki), (vc, vi)))
    del k, v
    from reskv_amd.tensors import CompressedKV, CompressedTensor

    def clone(ct):
        return CompressedTensor(ct.centroids.clone(), ct.cluster_ids.clone(), ct.payload.clone(),
                                None if ct.metadata is None else ct.metadata.clone(),
                                None if ct.scale is None else ct.scale.clone(), ct.plan)

    caches = [base] + [CompressedKV(clone(base.key), clone(base.value)) for _ in range(layers - 1)]
    q = torch.randn(b, HQ, 1, D, device=device, dtype=torch.float16)
    return caches, q


def time_steps(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / 1e3  # seconds


def measure_point(torch, b, t, sparsity, layout, layers, steps, warmup, device):
    from reskv_amd import attention

    caches, q = build_caches(torch, b, t, sparsity, layout, layers, device)
    freq = (500000.0 ** (-torch.arange(64, device=device).float() / 64)).float()
    pos = t

    def step():
        for c in caches:
            attention(q, c, position=pos, inv_freq=freq)

    secs = time_steps(torch, step, steps, warmup)
    plan = caches[0].key.plan
    nbytes = algorithmic_bytes(plan, b, t, caches[0].key.centroids.shape[2], caches[0].value.centroids.shape[2])
    per_call = secs / (steps * layers)
    del caches
    torch.cuda.empty_cache()
    return {
        "batch": b, "sparsity": sparsity, "layout": plan.layout, "fusion": plan.centroid_fusion,
        "seconds": secs, "us_per_layer_step": per_call * 1e6, "bytes_per_call": nbytes,
        "achieved_GBps": nbytes / per_call / 1e9, "frac": nbytes / per_call / HBM_PEAK,
        "tokens_per_s": b * steps / secs,
    }


def measure_dense(torch, b, t, layers, steps, warmup, device):
    from reskv_amd._extension import dense_decode

    torch.manual_seed(43)
    ks = [torch.randn(b, HK, t, D, device=device, dtype=torch.float16) * 0.5 for _ in range(min(layers, 4))]
    vs = [torch.randn_like(ks[0]) * 0.5 for _ in range(len(ks))]
    q = torch.randn(b, HQ, 1, D, device=device, dtype=torch.float16)
    freq = (500000.0 ** (-torch.arange(64, device=device).float() / 64)).float()
    n = len(ks)

    def step():
        for i in range(layers):
            dense_decode(q, ks[i % n], vs[i % n], freq, position=t)

    secs = time_steps(torch, step, steps, warmup)
    per_call = secs / (steps * layers)
    nbytes = algorithmic_bytes(None, b, t, 0, 0)
    del ks, vs
    torch.cuda.empty_cache()
    return {"batch": b, "us_per_layer_step": per_call * 1e6, "achieved_GBps": nbytes / per_call / 1e9,
            "frac": nbytes / per_call / HBM_PEAK, "caches": n}


def cpu_baseline(seconds_budget, b, t, sparsity):
    """numpy oracle decode (reconstruct + float64 attention) on one batch element."""
    import numpy as np

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import reskv_oracle as o

    rng = np.random.default_rng(42)
    nnz = int(128 * (1 - sparsity))
    k = (rng.standard_normal((1, HK, t, D)) * 0.5).astype(np.float16)
    v = (rng.standard_normal((1, HK, t, D)) * 0.5).astype(np.float16)
    kc = (rng.standard_normal((1, HK, 32, D)) * 0.1).astype(np.float16)
    vc = (rng.standard_normal((1, HK, 32, D)) * 0.1).astype(np.float16)
    ki = rng.integers(0, 32, (1, HK, t))
    vi = rng.integers(0, 32, (1, HK, t))
    kp, km = o.encode_bitmap(k, kc, ki, nnz)
    vp, vm = o.encode_bitmap(v, vc, vi, nnz)
    q = rng.standard_normal((1, HQ, 1, D)).astype(np.float16)
    f = o.theta_frequencies(500000.0)

    def one():
        kd = o.reconstruct("bitmap", kc, ki, kp, km)
        vd = o.reconstruct("bitmap", vc, vi, vp, vm)
        o.reference_attention(q, kd, vd, position=t, freq=f)

    one()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds_budget:
        one()
        n += 1
    per_elem = (time.perf_counter() - t0) / n
    cores = len(os.sched_getaffinity(0))
    # a decode step of the workload = LAYERS calls x b batch elements
    return {"value": 1.0 / (LAYERS * per_elem), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"numpy oracle: reconstruct + float64 attention, 1 batch element x {HK} KV heads x "
                      f"T={t}, bitmap {int(sparsity * 100)}% sparsity, {n} repetitions "
                      f"({per_elem * 1e3:.1f} ms each); tokens/s = 1 / ({LAYERS} layers x time per element)"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding is design-only "
                                   "(see DESIGN.md)", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    device = "cuda:0"
    torch.cuda.set_device(0)
    if args.sweep:
        for sparsity in (0.5, 0.75):
            for b in (1, 4, 8, 16, 32):
                r = measure_point(torch, b, args.seq_len, sparsity, args.layout, args.layers, args.steps,
                                  args.warmup, device)
                print(json.dumps({"sweep": r}), flush=True)
        for b in (1, 4, 8, 16, 32):
            print(json.dumps({"dense": measure_dense(torch, b, args.seq_len, args.layers, args.steps,
                                                     args.warmup, device)}), flush=True)
    r = measure_point(torch, args.batch, args.seq_len, args.sparsity, args.layout, args.layers, args.steps,
                      args.warmup, device)
    dense = measure_dense(torch, args.batch, args.seq_len, args.layers, max(2, args.steps // 4), 1, device)
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds, args.batch, args.seq_len, args.sparsity)
    secs = r["seconds"]
    line = {
        "metric": METRIC,
        "value": r["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": secs / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": f"config2 compressed-KV decode attention, {args.layers} layers x 1 decode step",
            "batch": args.batch, "seq_len": args.seq_len, "q_heads": HQ, "kv_heads": HK, "head_dim": D,
            "sparsity": args.sparsity, "layout": r["layout"], "centroid_fusion": r["fusion"],
            "storage": "fp16 residuals, int8 ids", "attn_us_per_layer_step": r["us_per_layer_step"],
            "dense_fp16_us_per_layer_step": dense["us_per_layer_step"],
            "speedup_vs_dense": dense["us_per_layer_step"] / r["us_per_layer_step"],
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm", "achieved": r["achieved_GBps"], "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": r["frac"], "traffic": None,
            "kernel": "decode_partial_kernel + decode_merge_kernel (one attention call)",
            "bytes_per_call": r["bytes_per_call"],
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
