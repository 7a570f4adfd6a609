"""Config 4 at its real shape: a random-init Llama-3.1-8B-shaped model (32
layers, hidden 4096, 32/8 heads, FFN 14336, vocab 128256, llama3 RoPE), an
8192-token random prompt at batch 16, compressed at prefill (75%, 32
clusters, 10 iterations, window 32, group 64), then greedy decode steps across
a group compression.  After the last step the final layer's attention output
is checked against the float64 oracle on a subset of (batch, KV head) pairs:
compressed history + the dense ring, with the model's llama3 frequencies."""

import numpy as np
import pytest
import torch

from oracle import reskv_oracle as o
from reskv_amd import ResKVKernelConfig
from reskv_amd.llama import GreedyDecoder, LlamaShape, RandomLlama
from tests.gpu_helpers import ATOL, np_, oracle_format

pytestmark = pytest.mark.gpu


def _dense_subset(ct, nb, nh):
    """Oracle reconstruction (float64) of batches [0, nb) and KV heads [0, nh)."""
    pick = lambda t: None if t is None else np_(t[:nb, :nh])  # noqa: E731
    return o.reconstruct(oracle_format(ct.plan), pick(ct.centroids), pick(ct.cluster_ids).astype(np.int64),
                         pick(ct.payload), pick(ct.metadata), pick(ct.scale), bits=ct.plan.bits)


def test_config4_decode_across_a_group_compression(device):
    shape = LlamaShape()
    batch, prompt, steps = 16, 8192, 40
    model = RandomLlama(shape, device, seed=0)
    ids = torch.randint(128, shape.vocab, (batch, prompt), generator=torch.Generator().manual_seed(42)).to(device)
    cfg = ResKVKernelConfig(sparsity=0.75, num_clusters=32, kmeans_iterations=10, recent_size=32, group_size=64)
    dec = GreedyDecoder(model, batch, prompt, steps + 1, "reskv", cfg)
    first = model.prefill(ids, dec.absorb)
    last = dec.caches[-1]
    assert last.compressed.seq_len == (prompt - 32) // 64 * 64 and last.live == prompt - last.compressed.seq_len
    dec.start(first)
    compressed_before = last.compressed.seq_len
    for _ in range(steps):
        tok = dec.step()
    torch.cuda.synchronize()
    assert last.compressed.seq_len == compressed_before + 64          # one group compressed during decode
    assert last.length == prompt + steps and last.compressed.key.centroids.shape[2] == 33
    assert bool(((tok >= 0) & (tok < shape.vocab)).all())
    # the last layer's attention of the last step: q, q_rot and attn still hold its values
    nb, nh, g = 2, 2, shape.heads // shape.kv_heads
    pos = prompt + steps - 1
    q = np_(dec.q[:nb, : nh * g]).astype(np.float64)[:, :, None]
    qr = np_(dec.qr[:nb, : nh * g]).astype(np.float64)[:, :, None]
    ring_k = np_(last.keys[:nb, :nh, : last.live]).astype(np.float64)
    ring_v = np_(last.values[:nb, :nh, : last.live]).astype(np.float64)
    ref = o.reference_attention(q, _dense_subset(last.compressed.key, nb, nh),
                                _dense_subset(last.compressed.value, nb, nh), position=pos,
                                freq=np_(model.inv_freq), scaling=model.scaling, recent=(qr, ring_k, ring_v))
    got = np_(dec.attn[:nb, : nh * g]).astype(np.float64)[:, :, None]
    assert np.abs(got - ref).max() <= ATOL
