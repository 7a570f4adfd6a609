"""Device-resident two-segment cache with the real compressor (GPU).

* The reference's incremental-cache invariants (reskv tests/test_cuda.py:74-89):
  no token lost and centroid tables capped.
* The capacity-buffer history equals, bit for bit, the chain the reference
  builds with ``compress(..., previous=...)`` and ``torch.cat``.
* Decode attention read in place from the capacity buffers (row-strided
  views), joined with the dense ring, matches the float64 oracle.
"""

import numpy as np
import pytest
import torch

from oracle import reskv_oracle as o
from reskv_amd import ResKVKernelConfig, attention, compress
from reskv_amd.cache import ResKVLayerCache
from tests.gpu_helpers import ATOL, expected_attention, np_, seeded

pytestmark = pytest.mark.gpu


def _inputs(t, device, seed=4, b=1, h=2):
    g = seeded(seed)
    k = (torch.randn(b, h, t, 128, generator=g) * 0.5).half().to(device)
    v = (torch.randn(b, h, t, 128, generator=g) * 0.5).half().to(device)
    return k, v


def test_incremental_cache_no_tokens_lost_and_centroids_capped(device):
    cfg = ResKVKernelConfig(bits=16, layout="unstructured", num_clusters=4, max_clusters=6, group_size=16,
                            recent_size=8)
    cache = ResKVLayerCache(cfg)
    k, v = _inputs(35, device)
    cache.update(k, v, {"raw_keys": k})
    assert cache.compressed.seq_len + cache.live == 35
    for _ in range(100):
        token = k[:, :, :1]
        cache.update(token, token, {"raw_keys": token})
        assert cache.compressed.seq_len + cache.live == cache.length
        assert cache.compressed.key.centroids.shape[2] <= 6
    assert cache.length == 135
    cache.reset()
    assert cache.get_seq_length() == 0 and cache.compressed is None


@pytest.mark.parametrize("bits,sparsity", [(16, 0.5), (16, 0.75), (4, 0.5), (2, 0.5)])
def test_capacity_history_equals_concatenated_chain(device, bits, sparsity):
    cfg = ResKVKernelConfig(bits=bits, sparsity=sparsity, num_clusters=8, max_clusters=12, group_size=32,
                            recent_size=16)
    k, v = _inputs(200, device, seed=6)
    layer = ResKVLayerCache(cfg, capacity=64)  # forces regrowth
    layer.update(k[:, :, :100], v[:, :, :100], {"raw_keys": k[:, :, :100]})
    for t in range(100, 200):
        layer.update(k[:, :, t:t + 1], v[:, :, t:t + 1], {"raw_keys": k[:, :, t:t + 1]})
    # the reference's chain: prefill compress, then one compress(previous=) per full ring
    n0 = (100 - 16) // 32 * 32
    ref = compress(k[:, :, :n0].contiguous(), v[:, :, :n0].contiguous(), cfg, plan=layer.plan)
    done = n0
    while done + 32 <= layer.compressed.seq_len:
        ref = compress(k[:, :, done:done + 32].contiguous(), v[:, :, done:done + 32].contiguous(), cfg,
                       previous=ref, plan=layer.plan)
        done += 32
    got = layer.compressed
    assert got.seq_len == ref.seq_len == done
    for a, b in ((got.key, ref.key), (got.value, ref.value)):
        assert torch.equal(a.centroids, b.centroids)
        assert torch.equal(a.cluster_ids, b.cluster_ids)
        assert torch.equal(a.payload, b.payload)
        assert (a.metadata is None) == (b.metadata is None)
        if a.metadata is not None:
            assert torch.equal(a.metadata, b.metadata)
        if a.scale is not None:
            assert torch.equal(a.scale, b.scale)


@pytest.mark.parametrize("bits,sparsity", [(16, 0.5), (16, 0.75), (4, 0.5)])
def test_decode_over_capacity_views_with_ring(device, bits, sparsity):
    cfg = ResKVKernelConfig(bits=bits, sparsity=sparsity, num_clusters=8, max_clusters=16, group_size=32,
                            recent_size=16)
    b, h, gqa = 2, 2, 4
    k, v = _inputs(260, device, seed=8, b=b, h=h)
    freq = (500000.0 ** (-torch.arange(64, device=device).float() / 64)).float()
    rot = lambda x, start: torch.from_numpy(  # noqa: E731
        o.rotate(np_(x).astype(np.float64), np.arange(start, start + x.shape[2]), np_(freq))).half().to(device)
    layer = ResKVLayerCache(cfg, capacity=96)
    layer.update(rot(k[:, :, :180], 0), v[:, :, :180], {"raw_keys": k[:, :, :180]})
    for t in range(180, 260):
        layer.update(rot(k[:, :, t:t + 1], t), v[:, :, t:t + 1], {"raw_keys": k[:, :, t:t + 1]})
    assert layer._k.ids.stride(1) > layer.compressed.seq_len  # a view with spare capacity
    q = torch.randn(b, h * gqa, 1, 128, generator=seeded(9)).half().to(device)
    pos = layer.length - 1
    qr = rot(q, pos)
    ring = (qr, layer.keys[:, :, : layer.live].contiguous(), layer.values[:, :, : layer.live].contiguous())
    out = attention(q, layer.compressed, position=pos, inv_freq=freq, recent=ring)
    ref = expected_attention(q, layer.compressed, position=pos, inv_freq=freq, recent=ring)
    assert float(np.abs(np_(out).astype(np.float64) - ref).max()) <= ATOL


@pytest.mark.parametrize("bits,sparsity", [(16, 0.5), (16, 0.75), (4, 0.5)])
def test_attend_fast_path_equals_attention(device, bits, sparsity):
    """layer.attend (cached descriptors, ring read in place) == attention(..., recent=ring), across group
    compressions that change the history."""
    cfg = ResKVKernelConfig(bits=bits, sparsity=sparsity, num_clusters=8, max_clusters=12, group_size=32,
                            recent_size=16)
    k, v = _inputs(220, device, seed=9, b=2, h=2)
    g = seeded(10)
    freq = (500000.0 ** (-torch.arange(64).float() / 64)).to(device)
    layer = ResKVLayerCache(cfg)
    layer.update(k[:, :, :120], v[:, :, :120], {"raw_keys": k[:, :, :120]})
    for t in range(120, 220):
        layer.update(k[:, :, t:t + 1], v[:, :, t:t + 1], {"raw_keys": k[:, :, t:t + 1]})
        if t % 7:
            continue
        q = torch.randn(2, 8, 1, 128, generator=g).half().to(device)
        qr = torch.randn(2, 8, 1, 128, generator=g).half().to(device)
        fast = layer.attend(q, qr, scaling=0.1, inv_freq=freq).clone()
        ref = attention(q, layer.compressed, position=layer.length - 1, inv_freq=freq, scaling=0.1,
                        recent=(qr, layer.keys[:, :, :layer.live], layer.values[:, :, :layer.live]))
        assert torch.equal(fast, ref), t


@pytest.mark.parametrize("sparsity,ring_len", [(0.5, 0), (0.5, 96), (0.75, 200)])
def test_step_decoder_one_merge_launch_equals_two(device, sparsity, ring_len):
    """reskv_decode_recent (the recent window joined inside the split merge) is bitwise
    decode + reskv_merge_recent_qk, including windows of more than one 128-token chunk,
    row-strided ring buffers and a caller-provided output buffer."""
    from reskv_amd._extension import StepDecoder

    k, v = _inputs(512, device, seed=21, b=2, h=2)
    cache = compress(k, v, ResKVKernelConfig(sparsity=sparsity, num_clusters=8))
    g = seeded(22)
    stride = max(ring_len, 1) + 8
    ring_k = (torch.randn(2, 2, stride, 128, generator=g) * 0.5).half().to(device)
    ring_v = (torch.randn(2, 2, stride, 128, generator=g) * 0.5).half().to(device)
    q = torch.randn(2, 8, 1, 128, generator=g).half().to(device)
    qr = torch.randn(2, 8, 1, 128, generator=g).half().to(device)
    freq = (500000.0 ** (-torch.arange(64).float() / 64)).to(device)
    step = StepDecoder(cache, 8, 0.1, freq)
    out = torch.full((2, 8, 1, 128), float("nan"), dtype=torch.float16, device=device)
    pos = 512 + ring_len
    got = step.run(q, pos, qr, ring_k, ring_v, ring_len, stride, out=out)
    assert got.data_ptr() == out.data_ptr()
    recent = None if ring_len == 0 else (qr, ring_k[:, :, :ring_len], ring_v[:, :, :ring_len])
    ref = attention(q, cache, position=pos, inv_freq=freq, scaling=0.1, recent=recent)
    assert torch.equal(out, ref)
    again = step.run(q, pos, qr, ring_k, ring_v, ring_len, stride)
    assert torch.equal(again, ref)


def test_decode_recent_with_empty_window_reads_no_recent_pointers(device):
    """reskv_decode_recent with Tr = 0 accepts null recent pointers (the C ABI's
    check) and must not read them: the result is the compressed-only decode."""
    import ctypes

    from reskv_amd import _lib
    from reskv_amd._extension import _rope, cache_descriptors

    k, v = _inputs(384, device, seed=31, b=2, h=2)
    cache = compress(k, v, ResKVKernelConfig(sparsity=0.5, num_clusters=8))
    g = seeded(32)
    q = torch.randn(2, 8, 1, 128, generator=g).half().to(device)
    freq = (500000.0 ** (-torch.arange(64).float() / 64)).to(device)
    kd, vd, keep = cache_descriptors(cache)
    f, table = _rope(freq, 500000.0, q.device, 384)
    L = _lib.lib()
    out = torch.full((2 * 8, 128), float("nan"), dtype=torch.float16, device=device)
    ws = torch.empty(L.reskv_decode_workspace_bytes(2, 8, 2, 384, 0), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    _lib.check(L.reskv_decode_recent(q.data_ptr(), ctypes.byref(kd), ctypes.byref(vd), f.data_ptr(), table.data_ptr(),
                                     2, 8, 2, 384, 0, 390, 0.1, 0, None, None, None, 0, 0, out.data_ptr(),
                                     ws.data_ptr(), ws.numel(), stream), "decode_recent")
    torch.cuda.synchronize()
    ref = attention(q, cache, position=390, inv_freq=freq, scaling=0.1)
    assert torch.equal(out.view(2, 8, 1, 128), ref)


def test_attend_with_a_ring_of_several_chunks(device):
    """recent_size 256 + group 64: the ring holds up to 320 tokens, read in place
    by the split merge's multi-chunk join; checked against the oracle."""
    cfg = ResKVKernelConfig(sparsity=0.5, num_clusters=8, max_clusters=12, group_size=64, recent_size=256)
    k, v = _inputs(700, device, seed=41, b=1, h=2)
    g = seeded(42)
    freq = (500000.0 ** (-torch.arange(64).float() / 64)).to(device)
    layer = ResKVLayerCache(cfg)
    layer.update(k[:, :, :400], v[:, :, :400], {"raw_keys": k[:, :, :400]})
    checked = 0
    for t in range(400, 700):
        layer.update(k[:, :, t:t + 1], v[:, :, t:t + 1], {"raw_keys": k[:, :, t:t + 1]})
        if layer.live <= 128 or t % 23:
            continue
        q = torch.randn(1, 8, 1, 128, generator=g).half().to(device)
        pos = layer.length - 1
        qr = torch.from_numpy(o.rotate(np_(q).astype(np.float64), np.array([pos]), np_(freq))).half().to(device)
        got = layer.attend(q, qr, scaling=128 ** -0.5, inv_freq=freq)
        ring = (qr, layer.keys[:, :, :layer.live], layer.values[:, :, :layer.live])
        ref = expected_attention(q, layer.compressed, position=pos, inv_freq=freq, recent=ring)
        assert float(np.abs(np_(got).astype(np.float64) - ref).max()) <= ATOL, t
        checked += 1
    assert checked >= 3
