"""Cache bookkeeping on the CPU (reskv/cache.py:11-122 semantics).

The compressor is replaced by a deterministic CPU stand-in that encodes each
token's position into its payload, so the tests can check which tokens went
into the compressed history, in what order, and with which centroid table,
without a GPU.  The real compressor is exercised by tests/test_gpu_cache.py.
"""

import pytest
import torch

import reskv_amd.cache as cache_mod
from reskv_amd import ResKVKernelConfig
from reskv_amd.cache import ResKVCache, ResKVLayerCache
from reskv_amd.tensors import CompressedKV, CompressedTensor

CFG = ResKVKernelConfig(bits=16, layout="unstructured", num_clusters=4, max_clusters=6, group_size=16,
                        recent_size=8)


def _fake_ct(x, plan, nc):
    """Payload[..., 0] carries the token's first channel; ids cycle; bitmaps select channels 0..nnz-1."""
    b, h, t, _ = x.shape
    cent = torch.full((b, h, nc, 128), float(nc), dtype=torch.float16)
    ids = (torch.arange(t) % nc).to(torch.int8).expand(b, h, t).contiguous()
    payload = x[..., : plan.nnz].clone()
    meta = torch.full((b, h, t, 2), -1, dtype=torch.int64)
    return CompressedTensor(cent, ids, payload, meta, None, plan)


def _install_fakes(monkeypatch):
    calls = {"fresh": 0, "group": 0}

    def fake_compress(k, v, config, *, previous=None, plan=None, clustering=None):
        assert previous is None
        calls["fresh"] += 1
        nc = config.num_clusters
        return CompressedKV(_fake_ct(k, plan, nc), _fake_ct(v, plan, nc))

    def fake_group(k, v, config, previous, plan):
        calls["group"] += 1
        nc = min(previous.key.centroids.shape[2] + 1, config.max_clusters)
        return _fake_ct(k, plan, nc), _fake_ct(v, plan, nc)

    monkeypatch.setattr(cache_mod, "compress", fake_compress)
    monkeypatch.setattr(cache_mod, "_compress_group", fake_group)
    return calls


def _tokens(t, start=0, b=1, h=2):
    """Token i carries the value start + i in every channel."""
    x = (torch.arange(start, start + t, dtype=torch.float32)[None, None, :, None]).expand(b, h, t, 128)
    return x.to(torch.float16).contiguous()


def test_prefill_split_and_group_compression(monkeypatch):
    calls = _install_fakes(monkeypatch)
    layer = ResKVLayerCache(CFG, capacity=32)
    x = _tokens(35)
    ring_k, _ = layer.update(x, x, {"raw_keys": x})
    # floor((35 - 8) / 16) * 16 = 16 compressed, 19 dense
    assert layer.compressed.seq_len == 16 and layer.live == 19 and layer.length == 35
    assert torch.equal(ring_k[0, 0, :, 0], torch.arange(16, 35, dtype=torch.float16))
    for step in range(100):
        y = _tokens(1, start=35 + step)
        layer.update(y, y, {"raw_keys": y})
        assert layer.compressed.seq_len + layer.live == layer.length
        assert layer.compressed.key.centroids.shape[2] <= CFG.max_clusters
        assert layer.live <= CFG.recent_size + CFG.group_size
    assert layer.length == 135 and calls["fresh"] == 1
    # every compressed token is present once, in order (payload channel 0 = position)
    kept = layer.compressed.key.payload[0, 0, :, 0].float()
    assert torch.equal(kept, torch.arange(kept.numel(), dtype=torch.float32))
    ring = layer.keys[0, 0, : layer.live, 0].float()
    assert torch.equal(ring, torch.arange(kept.numel(), 135, dtype=torch.float32))
    # one centroid appended per group until the cap
    assert layer.compressed.key.centroids.shape[2] == min(4 + calls["group"], 6)


def test_capacity_grows_without_losing_tokens(monkeypatch):
    _install_fakes(monkeypatch)
    layer = ResKVLayerCache(CFG, capacity=1)
    x = _tokens(40)
    layer.update(x, x, {"raw_keys": x})
    for step in range(300):
        y = _tokens(1, start=40 + step)
        layer.update(y, y, {"raw_keys": y})
    n = layer.compressed.seq_len
    assert layer._k.capacity >= n
    assert torch.equal(layer.compressed.value.payload[0, 1, :, 5].float(), torch.arange(n, dtype=torch.float32))


def test_short_prompt_starts_compressing_at_first_full_ring(monkeypatch):
    calls = _install_fakes(monkeypatch)
    layer = ResKVLayerCache(CFG)
    x = _tokens(10)
    layer.update(x, x, {"raw_keys": x})
    assert layer.compressed is None and layer.live == 10
    for step in range(14):
        y = _tokens(1, start=10 + step)
        layer.update(y, y, {"raw_keys": y})
    assert layer.compressed is not None and calls["fresh"] == 1
    assert layer.compressed.seq_len == 16 and layer.live == 8


def test_views_share_the_capacity_buffers(monkeypatch):
    _install_fakes(monkeypatch)
    layer = ResKVLayerCache(CFG, capacity=64)
    x = _tokens(40)
    layer.update(x, x, {"raw_keys": x})
    ids = layer.compressed.key._native[1]
    assert ids.data_ptr() == layer._k.ids.data_ptr() and ids.stride(0) == 64


def test_validation_and_reset(monkeypatch):
    _install_fakes(monkeypatch)
    layer = ResKVLayerCache(CFG)
    x = _tokens(40)
    with pytest.raises(ValueError, match="raw_keys"):
        layer.update(x, x)
    layer.update(x, x, {"raw_keys": x})
    with pytest.raises(ValueError, match="one token per step"):
        layer.update(x[:, :, :2], x[:, :, :2], {"raw_keys": x[:, :, :2]})
    assert layer.get_mask_sizes(3) == (43, 0)
    layer.reset()
    assert layer.get_seq_length() == 0 and layer.compressed is None and not layer.is_initialized


def test_reorder_and_crop(monkeypatch):
    _install_fakes(monkeypatch)
    c = ResKVCache(CFG, num_layers=2)
    x = torch.cat((_tokens(40, b=1), _tokens(40, start=100, b=1)), 0)
    for layer in c.layers:
        layer.update(x, x, {"raw_keys": x})
    c.reorder_cache(torch.tensor([1, 1]))
    for layer in c.layers:
        assert torch.equal(layer.compressed.key.payload[0], layer.compressed.key.payload[1])
        assert float(layer.compressed.key.payload[0, 0, 0, 0]) == 100.0
    with pytest.raises(NotImplementedError):
        c.crop(3)
    assert c.get_seq_length() == 40 and len(c) == 2
