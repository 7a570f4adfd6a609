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


def _small_llama():
    return LlamaConfig(hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=4,
                       num_key_value_heads=1, vocab_size=256, max_position_embeddings=8192, rope_theta=500000.0)


@pytest.mark.parametrize("bits,sparsity", [(16, 0.5), (16, 0.75), (4, 0.5), (4, 0.75), (2, 0.5)])
def test_plans_through_generate_and_save_reload(device, tmp_path, monkeypatch, bits, sparsity):
    """Every residual format through transformers' generate across group
    compressions, then save/reload with equal logits (reskv tests/test_model.py:29-58:
    96-token prompt, recent window 16, groups of 32, 4 clusters of at most 8, 66 new
    tokens, i.e. two group compressions after the prefill split).  The attention the
    model computes over the compressed history is checked against the float64
    oracle at the first decode steps and after each group compression."""
    torch.manual_seed(9)
    settings = ResKVKernelConfig(bits=bits, sparsity=sparsity, layout="auto", recent_size=16, group_size=32,
                                 num_clusters=4, max_clusters=8)
    model = ResKVForCausalLM(_small_llama(), settings).cuda().half().eval()
    checked = []  # (compressed length, position, max-abs error against the oracle)
    first_layer = []
    original = ResKVLayerCache.attend

    def recording(self, query, query_rot, *, scaling, inv_freq=None, rope_theta=500000.0):
        out = original(self, query, query_rot, scaling=scaling, inv_freq=inv_freq, rope_theta=rope_theta)
        if not first_layer:
            first_layer.append(self)  # the first attend of a decode step is layer 0's
        comp = self.compressed
        if self is first_layer[0] and (len(checked) < 2 or checked[-1][0] != comp.seq_len):
            assert comp.key.plan == settings.resolve(1)
            ring = (query_rot, self.keys[:, :, : self.live], self.values[:, :, : self.live])
            ref = expected_attention(query, comp, position=self.length - 1, inv_freq=inv_freq, scaling=scaling,
                                     recent=ring)
            checked.append((comp.seq_len, self.length - 1, float(abs(np_(out).astype("float64") - ref).max())))
        return out

    monkeypatch.setattr(ResKVLayerCache, "attend", recording)
    x = torch.randint(10, 200, (1, 96), device=device)
    with torch.inference_mode():
        initial = model(x, use_cache=True)
        cache = initial.past_key_values
        assert cache.layers[0].compressed.key.plan == settings.resolve(1)
        result = model.generate(x, max_new_tokens=66, do_sample=False, eos_token_id=None, pad_token_id=0)
    assert result.shape == (1, 162)
    assert len({c[0] for c in checked}) >= 3  # the prefill split and two group compressions
    for length, position, err in checked:
        assert err <= ATOL, (length, position, err)
    model.save_pretrained(tmp_path)
    restored = ResKVForCausalLM.from_pretrained(tmp_path, dtype=torch.float16).cuda().eval()
    assert restored.kernel_config == settings
    assert restored.config.reskv_kernel_config == settings.to_dict()
    with torch.inference_mode():
        torch.testing.assert_close(initial.logits, restored(x, use_cache=True).logits)
