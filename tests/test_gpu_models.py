"""Model patch on MI355X: a prompt long enough to compress, greedy generation
through transformers' ``generate``, cache bookkeeping, and the attention the
model computes over the compressed history checked against the float64 oracle."""

import pytest
import torch

pytest.importorskip("transformers")
from transformers import LlamaConfig  # noqa: E402

from reskv_amd import ResKVForCausalLM, ResKVKernelConfig  # noqa: E402
from reskv_amd.cache import ResKVLayerCache  # noqa: E402
from tests.gpu_helpers import ATOL, expected_attention, np_  # noqa: E402

pytestmark = pytest.mark.gpu


def _model(sparsity, rope_parameters=None):
    kw = dict(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=4,
              num_key_value_heads=1, max_position_embeddings=8192)
    if rope_parameters is not None:
        kw["rope_parameters"] = rope_parameters
    torch.manual_seed(7)
    cfg = ResKVKernelConfig(sparsity=sparsity, num_clusters=8, kmeans_iterations=4)
    return ResKVForCausalLM(LlamaConfig(**kw), cfg).half().cuda().eval()


@pytest.mark.parametrize("sparsity,rope", [
    (0.5, None),
    (0.75, {"rope_type": "llama3", "rope_theta": 500000.0, "factor": 8.0, "low_freq_factor": 1.0,
            "high_freq_factor": 4.0, "original_max_position_embeddings": 256}),
])
def test_generate_over_compressed_history(device, monkeypatch, sparsity, rope):
    model = _model(sparsity, rope)
    seen = []
    original = ResKVLayerCache.attend

    def recording(self, query, query_rot, *, scaling, inv_freq=None, rope_theta=500000.0):
        out = original(self, query, query_rot, scaling=scaling, inv_freq=inv_freq, rope_theta=rope_theta)
        if self is model_cache().layers[0] and len(seen) < 3:
            ring = (query_rot.clone(), self.keys[:, :, : self.live].clone(), self.values[:, :, : self.live].clone())
            seen.append((query.clone(), self.compressed, self.length - 1, inv_freq, scaling, ring, out.clone()))
        return out

    monkeypatch.setattr(ResKVLayerCache, "attend", recording)
    caches = []
    model_cache = lambda: caches[-1]  # noqa: E731
    ids = torch.randint(10, 1000, (2, 200), generator=torch.Generator().manual_seed(3)).cuda()

    def first_forward_hook(module, args, kwargs, output):
        if not caches:
            caches.append(output.past_key_values)

    handle = model.register_forward_hook(first_forward_hook, with_kwargs=True)
    with torch.no_grad():
        out = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=40, do_sample=False,
                             pad_token_id=0)
    handle.remove()
    assert out.shape == (2, 240) and int(out.min()) >= 0 and int(out.max()) < 1000
    cache = caches[0]
    for layer in cache.layers:
        assert layer.get_seq_length() == 239  # the last generated token is not fed back
        assert layer.compressed.seq_len + layer.live == layer.get_seq_length()
        assert layer.compressed.seq_len >= 128 and layer.live <= 96
    assert len(seen) == 3
    for q, comp, position, freq, scaling, ring, got in seen:
        assert freq is not None and freq.dtype == torch.float32
        ref = expected_attention(q, comp, position=position, inv_freq=freq, scaling=scaling, recent=ring)
        assert float(abs(np_(got).astype("float64") - ref).max()) <= ATOL
