"""Decode-attention benchmark over the compressed KV cache on one MI355X.

Workload (Llama-3.1-8B layer shape): 32 query heads,
8 KV heads, head_dim 128, RoPE theta 500000, compressed context T = 8192,
synthetic KV following reskv benchmarks/kernels.py:57-65 (k, v ~ 0.5 N(0,1),
centroids ~ 0.1 N(0,1), random cluster ids, seed 42).  One *step* is one
decode step of a 32-layer model: 32 fused decode-attention calls, each on its
own layer cache (32 distinct caches, so the 256 MB Infinity Cache cannot hold
the working set).  The step is captured once in a HIP graph and replayed, so
the timed region holds only GPU work (the eager, Python-dispatched time per
call is reported next to it).  ``value`` = batch * steps / elapsed (tokens/s).

The JSON line also carries the roofline of one decode-attention call
(algorithmic compressed bytes per call / measured time per call vs 8 TB/s),
a sweep over the batch sizes and sparsities of config 2 plus the dense fp16
baseline at the same shapes (this build's dense HIP kernel, and torch's
scaled_dot_product_attention for reference), config 1 (prefill compression), config 3
(INT4/INT2 decode), a stated-length config-4 end-to-end decode (ResKV against
dense fp16 KV), and a CPU baseline: the torch restatement of the reference's
compress and attention (oracle/torch_checker.py) on this host's cores.
"""

import argparse
import json
import os
import sys
import time

HBM_PEAK = 8.0e12  # bytes/s, MI355X HBM3E
FP16_MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 matrix-core peak of an MI355X
METRIC = "decode tok/s, Llama-3.1-8B-shape 8K ctx bs1-32; attn µs/step + % HBM peak"
LAYERS = 32
HQ, HK, D, T = 32, 8, 128, 8192
BATCHES = (1, 4, 8, 16, 32)


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
    p.add_argument("--splits", type=int, default=0, help="split-K count (0: automatic)")
    p.add_argument("--no-sweep", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-e2e", action="store_true", help="leave the config-4 end-to-end decode out of the line")
    p.add_argument("--e2e-steps", type=int, default=2048,
                   help="new tokens per sequence timed in the config-4 decode (config 4 names 2048)")
    p.add_argument("--e2e-batch", type=int, default=16)
    p.add_argument("--e2e-prompt", type=int, default=8192)
    p.add_argument("--only", choices=("encode", "quantized", "e2e"), default=None,
                   help="run just the config 1 (encode) or config 3 (quantized) measurement and print it")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="also run a 256 MiB device copy (reference point for HBM byte counters)")
    return p.parse_args()


def algorithmic_bytes(plan, b, t, nc_k, nc_v):
    """Compressed bytes one decode call must read (+ q read, out write).

    Per (batch, kv-head): T * (2 int8 ids + K/V payload + K/V metadata + K/V
    scales) + both centroid tables; per query head: q in, out written (fp16).
    """
    if plan is None:  # dense fp16
        per_tok = 2 * D * 2
        cent = 0
    else:
        if plan.bits == 16:
            payload, meta, scale = 2 * plan.nnz, 16, 0
        elif plan.layout == "structured":
            payload, meta, scale = 16, 8, 2
        else:
            payload, meta, scale = 4 * 4 * plan.bits, 0, 2
        per_tok = 2 * (1 + payload + meta + scale)
        cent = (nc_k + nc_v) * D * 2
    return b * HK * (t * per_tok + cent) + 2 * b * HQ * D * 2


def build_caches(torch, b, t, sparsity, layout, layers, device):
    from reskv_amd import ResKVKernelConfig, compress
    from reskv_amd.tensors import CompressedKV, CompressedTensor

    cfg = ResKVKernelConfig(sparsity=sparsity, layout=layout)
    g = torch.Generator(device=device).manual_seed(42)
    shape = (b, HK, t, D)
    k = torch.randn(shape, device=device, dtype=torch.float16, generator=g) * 0.5
    v = torch.randn(shape, device=device, dtype=torch.float16, generator=g) * 0.5
    kc = torch.randn(b, HK, 32, D, device=device, dtype=torch.float16, generator=g) * 0.1
    vc = torch.randn(b, HK, 32, D, device=device, dtype=torch.float16, generator=g) * 0.1
    ki = torch.randint(32, (b, HK, t), device=device, dtype=torch.int32, generator=g)
    vi = torch.randint(32, (b, HK, t), device=device, dtype=torch.int32, generator=g)
    base = compress(k, v, cfg, clustering=((kc, ki), (vc, vi)))
    del k, v

    def clone(ct):
        return CompressedTensor(ct.centroids.clone(), ct.cluster_ids.clone(), ct.payload.clone(),
                                None if ct.metadata is None else ct.metadata.clone(),
                                None if ct.scale is None else ct.scale.clone(), ct.plan)

    caches = [base] + [CompressedKV(clone(base.key), clone(base.value)) for _ in range(layers - 1)]
    q = torch.randn(b, HQ, 1, D, device=device, dtype=torch.float16, generator=g)
    return caches, q


def graph_time(torch, fn, steps, warmup):
    """Seconds for `steps` replays of a graph holding one call of fn()."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # eager warm-up outside the capture (library load, allocator)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    end.synchronize()
    del graph
    return start.elapsed_time(end) / 1e3


def eager_time(torch, fn, steps):
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def measure_point(torch, b, t, sparsity, layout, layers, steps, warmup, splits, device, eager=False):
    from reskv_amd import attention

    caches, q = build_caches(torch, b, t, sparsity, layout, layers, device)
    freq = (500000.0 ** (-torch.arange(64, device=device).float() / 64)).float()

    def step():
        for c in caches:
            attention(q, c, position=t, inv_freq=freq, splits=splits)

    secs = graph_time(torch, step, steps, warmup)
    per_call = secs / (steps * layers)
    out = {}
    if eager:
        out["eager_us_per_layer_step"] = eager_time(torch, step, max(2, steps // 4)) / (max(2, steps // 4) * layers) * 1e6
    plan = caches[0].key.plan
    nbytes = algorithmic_bytes(plan, b, t, caches[0].key.centroids.shape[2], caches[0].value.centroids.shape[2])
    from reskv_amd._extension import decode_splits

    nsplit = decode_splits(caches[0], HQ, splits)
    del caches
    torch.cuda.empty_cache()
    out.update({
        "batch": b, "sparsity": sparsity, "layout": plan.layout, "fusion": plan.centroid_fusion,
        "splits": nsplit, "seconds": secs, "us_per_layer_step": per_call * 1e6, "bytes_per_call": nbytes,
        "achieved_GBps": nbytes / per_call / 1e9, "frac": nbytes / per_call / HBM_PEAK,
        "tokens_per_s": b * steps / secs,
    })
    return out


def measure_dense(torch, b, t, layers, steps, warmup, device):
    from reskv_amd._extension import dense_decode

    g = torch.Generator(device=device).manual_seed(43)
    n = max(2, min(layers, (2 << 30) // (b * HK * t * D * 2 * 2)))  # distinct caches, >= 2 GB total
    ks = [torch.randn(b, HK, t, D, device=device, dtype=torch.float16, generator=g) * 0.5 for _ in range(n)]
    vs = [torch.randn(b, HK, t, D, device=device, dtype=torch.float16, generator=g) * 0.5 for _ in range(n)]
    q = torch.randn(b, HQ, 1, D, device=device, dtype=torch.float16, generator=g)
    freq = (500000.0 ** (-torch.arange(64, device=device).float() / 64)).float()

    def step():
        for i in range(layers):
            dense_decode(q, ks[i % n], vs[i % n], freq, position=t)

    secs = graph_time(torch, step, steps, warmup)
    per_call = secs / (steps * layers)
    nbytes = algorithmic_bytes(None, b, t, 0, 0)
    del ks, vs
    torch.cuda.empty_cache()
    return {"batch": b, "us_per_layer_step": per_call * 1e6, "achieved_GBps": nbytes / per_call / 1e9,
            "frac": nbytes / per_call / HBM_PEAK, "distinct_caches": n}


def measure_sdpa(torch, b, t, layers, steps, device):
    """torch's scaled_dot_product_attention on dense fp16 K/V (already rotated),
    a reference point beside the dense HIP kernel.  The four query heads of a
    KV head ride in the query-length axis ([B, 8, 4, 128] against [B, 8, T,
    128]), the same product as grouped-query decode with K/V read once.  Only
    the flash and memory-efficient backends are allowed; where neither takes
    the call the result says why instead of a time.  Timed eagerly (events
    around `steps` rounds of `layers` calls)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    g = torch.Generator(device=device).manual_seed(44)
    n = max(2, min(layers, (2 << 30) // (b * HK * t * D * 2 * 2)))
    ks = [torch.randn(b, HK, t, D, device=device, dtype=torch.float16, generator=g) * 0.5 for _ in range(n)]
    vs = [torch.randn(b, HK, t, D, device=device, dtype=torch.float16, generator=g) * 0.5 for _ in range(n)]
    q = torch.randn(b, HK, HQ // HK, D, device=device, dtype=torch.float16, generator=g)
    out = {"batch": b, "distinct_caches": n}

    def step():
        for i in range(layers):
            torch.nn.functional.scaled_dot_product_attention(q, ks[i % n], vs[i % n])

    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            step()
            torch.cuda.synchronize()
            secs = eager_time(torch, step, steps)
        per_call = secs / (steps * layers)
        nbytes = algorithmic_bytes(None, b, t, 0, 0)
        out.update({"us_per_layer_step": per_call * 1e6, "frac": nbytes / per_call / HBM_PEAK})
    except RuntimeError as e:
        out["error"] = str(e).splitlines()[0][:200]
    del ks, vs
    torch.cuda.empty_cache()
    return out


def measure_encoders(torch, device, reps=20):
    """prefill compression of one layer, B=1, 8 KV heads, T=8192.

    K-means (32 clusters, 10 iterations) over K and over V, then the residual
    encoders at 75% sparsity (structured 4:16 and forced-unstructured bitmaps).
    Encoder bytes = x + ids + centroid table read, payload + metadata written.
    K-means work = 2*T*C*D FLOP per head per iteration for the distances.
    Every figure is graph-replayed (GPU time of the launches, no Python
    dispatch in the timed region); one graph holds several calls so that the
    graph launch itself is amortised.
    """
    from reskv_amd._extension import load_extension
    from reskv_amd.compression import cluster, cluster_kv

    ext = load_extension("compression")
    g = torch.Generator(device=device).manual_seed(1)
    b, h, t = 1, HK, T
    scale = torch.exp(torch.randn(1, h, 1, D, device=device, generator=g))
    k = (torch.randn(b, h, t, D, device=device, generator=g) * scale).half()
    v = torch.randn(b, h, t, D, device=device, generator=g).half()

    def timed(fn, n=reps, inner=8):
        def calls():
            for _ in range(inner):
                fn()
        return graph_time(torch, calls, n, 2) / (n * inner) * 1e6  # us per call

    out = {}
    kc, ki = cluster(k, 32, 10)
    vc, vi = cluster(v, 32, 10, value=True)
    us_k = timed(lambda: cluster(k, 32, 10), max(3, reps // 4), 2)
    us_v = timed(lambda: cluster(v, 32, 10, value=True), max(3, reps // 4), 2)
    us_kv = timed(lambda: cluster_kv(k, v, 32, 10), max(3, reps // 4), 2)
    flop = 2.0 * t * 32 * D * h * 10
    # matrix-core work the kernels issue per iteration and head: K takes the
    # distance product twice (fp16 hi and lo parts of its fp32 centres), V once;
    # both add the one-hot member sums (2 T C D) and counts (2 T C 16)
    mfma_k = (6.0 * t * 32 * D + 2.0 * t * 32 * 16) * h * 10
    mfma_v = (4.0 * t * 32 * D + 2.0 * t * 32 * 16) * h * 10
    out["kmeans"] = {"us_k": us_k, "us_v": us_v, "us_kv_together": us_kv, "tflops_k": flop / us_k / 1e6,
                     "tflops_v": flop / us_v / 1e6, "iterations": 10, "clusters": 32,
                     "mfma_tflops_kv": (mfma_k + mfma_v) / us_kv / 1e6,
                     "mfma_util": (mfma_k + mfma_v) / us_kv / 1e6 / FP16_MFMA_PEAK_TFLOPS,
                     "algorithmic_frac_of_fp16_peak": 2 * flop / us_kv / 1e6 / FP16_MFMA_PEAK_TFLOPS,
                     "mfma_note": "mfma_util: fp16 matrix-core FLOP issued (K: hi and lo distance products, "
                                  "V: one; one-hot member sums and counts) per second of the paired K+V run, "
                                  "over the 2.5 PFLOP/s dense fp16 peak; algorithmic: the distance FLOP "
                                  "2 T C D alone"}
    n_in = b * h * t * (D * 2 + 4) + b * h * 32 * D * 2
    # K and V encoded in one launch, as compress runs them
    cases = (("structured_fp16_75", 32 * 2 + 16, lambda: ext.compress_fp16_kv(k, kc, ki, v, vc, vi, 32, True)),
             ("bitmap_fp16_75", 32 * 2 + 16, lambda: ext.compress_bitmap_kv(k, kc, ki, v, vc, vi, 32)),
             ("bitmap_fp16_50", 64 * 2 + 16, lambda: ext.compress_bitmap_kv(k, kc, ki, v, vc, vi, 64)))
    for name, out_bytes, fn in cases:
        us = timed(fn)
        moved = 2 * (n_in + b * h * t * out_bytes)
        out[name] = {"us_kv": us, "GBps": moved / us / 1e3, "frac": moved / us / 1e3 / (HBM_PEAK / 1e9),
                     "launches": 1}
    del k, v
    torch.cuda.empty_cache()
    return out


def measure_quantized(torch, device, steps, layers=32):
    """INT4 / INT2 unstructured residuals at T=16384, B=8, 50% sparsity."""
    out = {}
    for bits in (4, 2):
        r = measure_point_bits(torch, 8, 16384, bits, layers, steps, device)
        out[f"int{bits}"] = r
    return out


def measure_point_bits(torch, b, t, bits, layers, steps, device):
    from reskv_amd import ResKVKernelConfig, attention, compress
    from reskv_amd.tensors import CompressedKV, CompressedTensor

    cfg = ResKVKernelConfig(sparsity=0.5, bits=bits)
    g = torch.Generator(device=device).manual_seed(3)
    k = torch.randn(b, HK, t, D, device=device, dtype=torch.float16, generator=g) * 0.5
    v = torch.randn(b, HK, t, D, device=device, dtype=torch.float16, generator=g) * 0.5
    kc = torch.randn(b, HK, 32, D, device=device, dtype=torch.float16, generator=g) * 0.1
    vc = torch.randn(b, HK, 32, D, device=device, dtype=torch.float16, generator=g) * 0.1
    ki = torch.randint(32, (b, HK, t), device=device, dtype=torch.int32, generator=g)
    vi = torch.randint(32, (b, HK, t), device=device, dtype=torch.int32, generator=g)
    base = compress(k, v, cfg, clustering=((kc, ki), (vc, vi)))
    del k, v

    def clone(ct):
        return CompressedTensor(ct.centroids.clone(), ct.cluster_ids.clone(), ct.payload.clone(), None,
                                ct.scale.clone(), ct.plan)

    caches = [base] + [CompressedKV(clone(base.key), clone(base.value)) for _ in range(layers - 1)]
    q = torch.randn(b, HQ, 1, D, device=device, dtype=torch.float16, generator=g)
    freq = (500000.0 ** (-torch.arange(64, device=device).float() / 64)).float()

    def step():
        for c in caches:
            attention(q, c, position=t, inv_freq=freq)

    secs = graph_time(torch, step, steps, 2)
    per_call = secs / (steps * layers)
    nbytes = algorithmic_bytes(base.key.plan, b, t, 32, 32)
    from reskv_amd._extension import decode_splits

    nsplit = decode_splits(caches[0], HQ)
    del caches
    torch.cuda.empty_cache()
    frac = nbytes / per_call / HBM_PEAK
    rec = counter_record(b, t, 0.5, "unstructured", bits)
    traffic, source = measured_traffic(rec, nsplit)
    return {"us_per_layer_step": per_call * 1e6, "achieved_GBps": nbytes / per_call / 1e9,
            "frac": frac, "splits": nsplit, "bytes_per_call": nbytes, "traffic": traffic,
            "traffic_ratio": traffic / nbytes if traffic else None, "traffic_source": source,
            "ceiling": issue_ceiling(rec, nbytes, frac)}


def measure_e2e(torch, device, batch=16, prompt=8192, steps=2048, warmup=4, attn_steps=8):
    """Config 4: greedy decode of a random-init Llama-3.1-8B-shaped model (32 layers,
    hidden 4096, 32/8 heads, FFN 14336, vocab 128256, llama3 RoPE theta 500000) at
    batch 16 after an 8192-token random prompt, with the ResKV cache (75%, 32
    clusters, 10 iterations, window 32, group 64) and with dense fp16 KV.  Reports
    decode tok/s, TPOT and the attention share of the step time."""
    from reskv_amd import ResKVKernelConfig
    from reskv_amd.llama import GreedyDecoder, LlamaShape, RandomLlama

    shape = LlamaShape()
    model = RandomLlama(shape, device, seed=0)
    ids = torch.randint(128, shape.vocab, (batch, prompt), generator=torch.Generator().manual_seed(42)).to(device)
    cfg = ResKVKernelConfig(sparsity=0.75, num_clusters=32, kmeans_iterations=10, recent_size=32, group_size=64)
    total = warmup + steps + attn_steps
    decs = {"reskv": GreedyDecoder(model, batch, prompt, total, "reskv", cfg),
            "dense_fp16": GreedyDecoder(model, batch, prompt, total, "dense")}

    compress_events = []

    def sink(layer, raw_k, rot_k, v):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        decs["reskv"].absorb(layer, raw_k, rot_k, v)  # K-means, encoders, ring copy of this layer
        e1.record()
        compress_events.append((e0, e1))
        decs["dense_fp16"].absorb(layer, raw_k, rot_k, v)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    first = model.prefill(ids, sink)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    compress_ms = [a.elapsed_time(b) for a, b in compress_events]
    out = {"prefill_s_incl_compression": prefill_s,
           "prefill_compression_ms_per_layer": sum(compress_ms) / len(compress_ms),
           "prefill_compression_s_total": sum(compress_ms) / 1e3,
           "prefill_s_without_compression": prefill_s - sum(compress_ms) / 1e3,
           "prefill_compression_note": "GPU time between events around each layer's ResKV cache hand-off "
                                       "(K-means of K and V, residual encoders, ring copy) during the prompt "
                                       "forward; the dense cache's copy is outside it",
           "batch": batch, "prompt": prompt,
           "new_tokens_timed": steps, "config4_new_tokens": 2048,
           "note": (f"decode rates timed over {steps} greedy tokens after {warmup} warm-up tokens"
                    + ("" if steps == 2048 else f" (config 4 names 2048; the per-token work is the same, "
                                                 f"the history {prompt}+{steps})")),
           "model": "random-init Llama-3.1-8B shape (fp16 weights)"}
    for name, dec in decs.items():
        dec.start(first)
        dec.capture()
        for _ in range(warmup):
            dec.step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(steps):
            dec.step()
        torch.cuda.synchronize()
        secs = time.perf_counter() - t1
        events = []
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(attn_steps):
            dec.step(events)
        s1.record()
        torch.cuda.synchronize()
        step_ms = s0.elapsed_time(s1) / attn_steps
        attn_ms = sum(a.elapsed_time(b) for a, b in events) / attn_steps
        out[name] = {"tok_per_s": batch * steps / secs, "tpot_ms": secs / steps * 1e3,
                     "attention_ms_per_step": attn_ms, "step_ms_timed_with_events": step_ms,
                     "attention_share": attn_ms / step_ms}
        if name == "reskv":
            out[name]["cache_mb_per_layer"] = _reskv_cache_mb(dec)
    out["speedup_tok_per_s"] = out["reskv"]["tok_per_s"] / out["dense_fp16"]["tok_per_s"]
    return out


def _reskv_cache_mb(dec):
    layer = dec.caches[0]
    c = layer.compressed
    n = sum(x.numel() * x.element_size() for t in (c.key, c.value)
            for x in (t.centroids, t.cluster_ids, t.payload, t.metadata, t.scale) if x is not None)
    ring = 3 * layer.keys.numel() * layer.keys.element_size()
    return {"compressed": n / 1e6, "ring": ring / 1e6,
            "dense_fp16_same_length": 2 * dec.batch * 8 * layer.length * 128 * 2 / 1e6}


def cpu_baseline():
    """The reference's CPU path restated with torch (oracle/torch_checker.py,
    pinned to the numpy oracle and its golden vectors): ``compress`` (K-means
    + residual encode) and reference attention over the reconstruction, on
    this host's cores, 1 warm-up then the median of 3.  Bounded samples:

    * config 0: B = 1, 8 KV heads, T = 960 compressed (15 K-means iterations,
      50% bitmap) + attention with 64 dense sink/recent tokens -- in full;
    * config 1: compress of one layer, 8 heads x 8192 tokens, 10 iterations,
      75% structured -- in full;
    * config 2: attention at T = 8192, 50% bitmap on 4 of the 32 batch
      elements, scaled by 8 to B = 32 (time is linear in B);
    * config 3: attention at T = 16384, INT4 and INT2, 1 of the 8 batch
      elements, scaled by 8.

    ``value`` is the config-2 decode rate in the metric's unit: B = 32 tokens
    per 32-layer step.
    """
    import statistics

    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import torch_checker as tc
    from reskv_amd.config import KernelPlan
    from reskv_amd.tensors import CompressedKV, CompressedTensor

    cores = max(1, min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "16") or 16)))
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(42)

    def median3(fn):
        fn()
        runs = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            runs.append(time.perf_counter() - t0)
        return statistics.median(runs)

    def outlier_k(b, t):
        scale = torch.exp(torch.randn(1, HK, 1, D, generator=gen))
        scale[..., :4] *= 10.0
        return (torch.randn(b, HK, t, D, generator=gen) * scale).half()

    def cache_of(b, t, fmt, bits=16):
        x = (torch.randn(b, HK, t, D, generator=gen) * 0.5).half()
        c = (torch.randn(b, HK, 32, D, generator=gen) * 0.1).half()
        ids = torch.randint(32, (b, HK, t), generator=gen, dtype=torch.int32)
        if fmt == "bitmap":
            p, m = tc.encode_bitmap(x, c, ids, 64)
            ct = CompressedTensor(c, ids, p, m, None, KernelPlan("unstructured", "deferred", 16, 64, 2, 0))
        else:
            p, sc = tc.encode_multibit(x, c, ids, 64, bits)
            ct = CompressedTensor(c, ids, p, None, sc, KernelPlan("unstructured", "per_token", bits, 64, 16, 0))
        return CompressedKV(ct, ct)

    out = {}
    # config 0
    k0, v0 = outlier_k(1, 1024), torch.randn(1, HK, 1024, D, generator=gen).half()
    q0 = torch.randn(1, HQ, 1, D, generator=gen).half()
    kc, vc = k0[:, :, 4:964].contiguous(), v0[:, :, 4:964].contiguous()

    def c0_compress():
        (a, ai), (b_, bi) = tc.kmeans(kc, 32, 15), tc.kmeans(vc, 32, 15, value=True)
        return tc.encode_bitmap(kc, a, ai, 64), tc.encode_bitmap(vc, b_, bi, 64), (a, ai, b_, bi)

    (kp, km), (vp, vm), (a, ai, b_, bi) = c0_compress()
    plan = KernelPlan("unstructured", "deferred", 16, 64, 2, 0)
    cache0 = CompressedKV(CompressedTensor(a, ai, kp, km, None, plan), CompressedTensor(b_, bi, vp, vm, None, plan))
    recent = (q0, k0[:, :, list(range(4)) + list(range(964, 1024))], v0[:, :, list(range(4)) + list(range(964, 1024))])
    out["config0"] = {"compress_s": median3(c0_compress),
                      "attention_s": median3(lambda: tc.attention(q0, cache0, position=1024, start_position=4,
                                                                  recent=recent))}
    # config 1
    k1, v1 = outlier_k(1, 8192), torch.randn(1, HK, 8192, D, generator=gen).half()

    def c1_compress():
        (a, ai), (b_, bi) = tc.kmeans(k1, 32, 10), tc.kmeans(v1, 32, 10, value=True)
        tc.encode_structured(k1, a, ai, 32)
        tc.encode_structured(v1, b_, bi, 32)

    out["config1"] = {"compress_s": median3(c1_compress)}
    # config 2 (4 of 32 batch elements)
    cache2 = cache_of(4, T, "bitmap")
    q2 = torch.randn(4, HQ, 1, D, generator=gen).half()
    per_call = median3(lambda: tc.attention(q2, cache2, position=T)) * 8
    out["config2_b32_s50"] = {"attention_s_per_layer_step": per_call, "sample": "4 of 32 batch elements, x8"}
    # config 3 (1 of 8 batch elements)
    for bits in (4, 2):
        cache3 = cache_of(1, 16384, "quant", bits)
        q3 = torch.randn(1, HQ, 1, D, generator=gen).half()
        out[f"config3_int{bits}"] = {"attention_s_per_layer_step": median3(
            lambda: tc.attention(q3, cache3, position=16384)) * 8, "sample": "1 of 8 batch elements, x8"}
        del cache3
    return {"value": 32 / (LAYERS * per_call), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": "torch CPU restatement of compress + reference attention (oracle/torch_checker.py), "
                      f"{cores} threads, 1 warm-up + median of 3 per item; value = config 2 (B=32, T=8192, "
                      "50% bitmap) decode tokens/s from 4 of 32 batch elements scaled x8, 32 layers per step",
            "configs": out}


def copy_bandwidth(torch, device, nbytes=1 << 30, reps=10):
    """GB/s of a plain device-to-device copy (bytes read + bytes written per
    second): the bandwidth a streaming kernel reaches on this box, reported
    beside the 8 TB/s spec-sheet peak."""
    src = torch.empty(nbytes, dtype=torch.uint8, device=device).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    end.synchronize()
    secs = start.elapsed_time(end) / 1e3
    del src, dst
    torch.cuda.empty_cache()
    return 2.0 * nbytes * reps / secs / 1e9


def counter_record(b, t, sparsity, layout, bits=16):
    """The committed rocprofv3 record of this workload's partial kernel
    (profiles/decode_traffic.json), or None.

    Each record holds the HBM bytes per launch from two rocprofv3 --pmc passes
    (FETCH_SIZE, WRITE_SIZE), each scaled by what the same counter reads for a
    device copy of known size, and the instructions per (token, KV-head) from
    three passes of SQ counters; the profiles under profiles/ hold the runs
    and their commands.  None of it is measured by this run.
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "decode_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    for w in rec.get("workloads", []):
        if (w.get("batch"), w.get("seq_len"), w.get("sparsity"), w.get("layout"), w.get("bits")) == \
                (b, t, sparsity, layout, bits):
            return dict(w, clock_ghz=rec.get("clock_ghz"), source=rec.get("source"))
    return None


def measured_traffic(rec, splits):
    """(HBM bytes per launch, where that figure comes from) from a counter record."""
    if rec is None:
        return None, None
    source = {"profile": rec["source"], "file": "profiles/decode_traffic.json",
              "measured_at_splits": rec["splits"], "this_run_splits": splits,
              "note": "copied from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE passes, not measured by this run"}
    return rec["fetch_bytes"] + rec["write_bytes"], source


def issue_ceiling(rec, bytes_per_call, frac):
    """The bandwidth fraction at which the partial kernel's vector ALU would be
    busy every cycle with the instructions it issues per (token, KV-head) --
    four SIMD cycles per wave64 VALU instruction, 1024 SIMDs at the recorded
    shader clock -- and the measured fraction of that ceiling."""
    if rec is None:
        return None
    cycles = 4.0 * rec["valu_per_unit"]
    seconds = rec["units"] * cycles / (1024 * rec["clock_ghz"] * 1e9)
    ceil = bytes_per_call / seconds / HBM_PEAK
    return {"valu_per_unit": rec["valu_per_unit"], "mfma_per_unit": rec["mfma_per_unit"],
            "valu_issue_ceiling_frac": ceil, "frac_of_ceiling": frac / ceil,
            "basis": "VALU instructions per (token, KV-head) from the committed SQ counter passes "
                     f"(profiles/decode_traffic.json), 4 cycles each, 1024 SIMDs at {rec['clock_ghz']} GHz"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU sharding is a design note only, "
                                   "so --gpus above 1 is not supported", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    device = "cuda:0"
    torch.cuda.set_device(0)
    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=device).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only == "encode":
        print(json.dumps({"encode": measure_encoders(torch, device)}), flush=True)
        return
    if args.only == "quantized":
        print(json.dumps({"quantized": measure_quantized(torch, device, max(5, args.steps // 2))}), flush=True)
        return
    if args.only == "e2e":
        print(json.dumps({"e2e": measure_e2e(torch, device, args.e2e_batch, args.e2e_prompt, args.e2e_steps)}),
              flush=True)
        return
    r = measure_point(torch, args.batch, args.seq_len, args.sparsity, args.layout, args.layers, args.steps,
                      args.warmup, args.splits, device, eager=True)
    print(json.dumps({"point": r}), flush=True)
    sweep, dense, sdpa = [], [], []
    if not args.no_sweep:
        for sparsity in (0.5, 0.75):
            for b in BATCHES:
                s = measure_point(torch, b, args.seq_len, sparsity, args.layout, args.layers,
                                  max(5, args.steps // 2), 2, args.splits, device)
                sweep.append({k: s[k] for k in ("batch", "sparsity", "layout", "splits", "us_per_layer_step",
                                                "achieved_GBps", "frac")})
                print(json.dumps({"sweep": s}), flush=True)
        for b in BATCHES:
            d = measure_dense(torch, b, args.seq_len, args.layers, max(5, args.steps // 2), 2, device)
            dense.append(d)
            print(json.dumps({"dense": d}), flush=True)
        for b in BATCHES:
            d = measure_sdpa(torch, b, args.seq_len, args.layers, max(3, args.steps // 4), device)
            sdpa.append(d)
            print(json.dumps({"torch_sdpa": d}), flush=True)
    encode = quant = None
    if not args.no_sweep:
        encode = measure_encoders(torch, device)
        print(json.dumps({"encode": encode}), flush=True)
        quant = measure_quantized(torch, device, max(5, args.steps // 2))
        print(json.dumps({"quantized": quant}), flush=True)
    dense_b = next((d for d in dense if d["batch"] == args.batch), None)
    if dense_b is None:
        dense_b = measure_dense(torch, args.batch, args.seq_len, args.layers, max(5, args.steps // 2), 2, device)
    e2e = None
    if not args.no_e2e:
        e2e = measure_e2e(torch, device, args.e2e_batch, args.e2e_prompt, args.e2e_steps)
        print(json.dumps({"e2e": e2e}), flush=True)
    copy_gbps = copy_bandwidth(torch, device)
    cpu = None if args.no_cpu_baseline else cpu_baseline()
    rec = counter_record(args.batch, args.seq_len, args.sparsity, r["layout"])
    traffic, traffic_source = measured_traffic(rec, r["splits"])
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
        "dtype": "fp32+fp16",
        "data": "synthetic",
        "config": {
            "workload": f"config 2 compressed-KV decode attention, one decode step = {args.layers} layer calls "
                        f"(graph-replayed), batch {args.batch}, T={args.seq_len}, sparsity {args.sparsity}",
            "batch": args.batch, "seq_len": args.seq_len, "q_heads": HQ, "kv_heads": HK, "head_dim": D,
            "sparsity": args.sparsity, "layout": r["layout"], "centroid_fusion": r["fusion"],
            "splits": r["splits"],
            "storage": "fp16 centroids and residuals, int8 cluster ids, int64 bitmaps",
            "arithmetic": "fp32 RoPE, scores (v_mfma_f32_4x4x1f32) and online softmax; the softmax weights "
                          "are rounded to fp16 for P x V and the cluster mass on v_mfma_f32_4x4x4f16 with "
                          "fp32 accumulation",
            "attn_us_per_layer_step": r["us_per_layer_step"],
            "eager_us_per_layer_step": r["eager_us_per_layer_step"],
            "dense_fp16_us_per_layer_step": dense_b["us_per_layer_step"],
            "speedup_vs_dense": dense_b["us_per_layer_step"] / r["us_per_layer_step"],
            "parallelism": "single GPU",
            "sweep": sweep,
            "dense_sweep": [{k: d[k] for k in ("batch", "us_per_layer_step", "frac")} for d in dense],
            "torch_sdpa_fp16_sweep": [{k: d[k] for k in ("batch", "us_per_layer_step", "frac", "error") if k in d}
                                      for d in sdpa],
            "config1_prefill_compression": encode,
            "config3_quantized_decode_b8_t16384": quant,
            "config4_end_to_end": e2e,
        },
        "roofline": {
            "bound": "hbm", "achieved": r["achieved_GBps"], "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": r["frac"], "traffic": traffic, "traffic_source": traffic_source,
            "ceiling": issue_ceiling(rec, r["bytes_per_call"], r["frac"]),
            "kernel": "one decode-attention call (decode_partial_kernel + decode_merge_kernel)",
            "bytes_per_call": r["bytes_per_call"],
            "copy_GBps": copy_gbps, "frac_of_copy": r["achieved_GBps"] / copy_gbps,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
