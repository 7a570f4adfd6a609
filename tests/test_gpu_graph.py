"""Decode attention captured in a HIP graph, as bench.py times it: every replay
gives the eager call's output bit for bit.  Between replays the program runs
eager decodes of other inputs (which reuse the library's kernels, the RoPE
table and torch's allocator) and synchronises, and the captured inputs are
overwritten in place and restored, so a replay that read stale memory or
depended on a first-replay-only state would show."""

import pytest
import torch

from reskv_amd import ResKVKernelConfig, attention, compress
from tests.gpu_helpers import outlier_kv, theta_freq

pytestmark = pytest.mark.gpu


def _cache(bits, sparsity, layout, seed):
    k, v, q = outlier_kv(2, 2, 900, seed=seed, gqa=4)
    cfg = ResKVKernelConfig(bits=bits, sparsity=sparsity, layout=layout, num_clusters=16)
    return compress(k, v, cfg), q


@pytest.mark.parametrize("bits,sparsity,layout", [(16, 0.5, "unstructured"), (16, 0.75, "structured"),
                                                  (4, 0.5, "unstructured"), (2, 0.5, "unstructured")])
def test_graph_replays_equal_the_eager_call(device, bits, sparsity, layout):
    cache, q = _cache(bits, sparsity, layout, seed=31)
    other, q2 = _cache(bits, sparsity, layout, seed=32)
    freq = theta_freq()
    position = 905
    eager = attention(q, cache, position=position, inv_freq=freq).clone()  # also builds the RoPE table

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        attention(q, cache, position=position, inv_freq=freq)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = attention(q, cache, position=position, inv_freq=freq)

    saved_q = q.clone()
    for replay in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), replay
        # eager work between replays: another cache, and the captured query
        # overwritten and restored in place
        attention(q2, other, position=position, inv_freq=freq)
        q.copy_(torch.randn_like(q))
        attention(q, cache, position=position, inv_freq=freq)
        q.copy_(saved_q)
        torch.cuda.synchronize()
    del graph


def test_graph_replays_of_the_prefill_compressor(device):
    """K-means of K and V together and the K+V encoders, captured as bench.py
    times them: every replay's centres, ids, payloads and metadata equal the
    eager call's (the kernels are deterministic)."""
    from reskv_amd._extension import load_extension
    from reskv_amd.compression import cluster_kv

    ext = load_extension("compression")
    k, v, _ = outlier_kv(1, 4, 1500, seed=33, gqa=4)
    (kc, ki), (vc, vi) = cluster_kv(k, v, 16, 5)
    steps = {
        "kmeans": lambda: cluster_kv(k, v, 16, 5),
        "tile4": lambda: ext.compress_fp16_kv(k, kc, ki, v, vc, vi, 32, True),
        "bitmap": lambda: ext.compress_bitmap_kv(k, kc, ki, v, vc, vi, 64),
    }

    def flat(x):
        return [y for z in x for y in (flat(z) if isinstance(z, (tuple, list)) else [z])]

    for name, fn in steps.items():
        eager = [t.clone() for t in flat(fn())]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = flat(fn())
        assert len(out) == len(eager) > 0
        for replay in range(3):
            graph.replay()
            torch.cuda.synchronize()
            for a, b in zip(out, eager):
                assert torch.equal(a, b), (name, replay)
            fn()  # eager work between replays
            torch.cuda.synchronize()
        del graph
