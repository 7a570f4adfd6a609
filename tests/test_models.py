"""Model patch (reskv/models/llama.py) on CPU: before the first group is
compressed every step attends densely, so greedy decoding must equal the stock
transformers Llama with the same weights; plus the constructor and forward
checks of the reference."""

import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig, LlamaForCausalLM  # noqa: E402

from reskv_amd import ResKVForCausalLM, ResKVKernelConfig  # noqa: E402
from reskv_amd.cache import ResKVCache  # noqa: E402


def _config(**kw):
    base = dict(vocab_size=300, hidden_size=512, intermediate_size=768, num_hidden_layers=2, num_attention_heads=4,
                num_key_value_heads=1, max_position_embeddings=2048)
    base.update(kw)
    return LlamaConfig(**base)


def test_uncompressed_decode_equals_stock_llama():
    torch.manual_seed(0)
    stock = LlamaForCausalLM(_config()).eval()
    model = ResKVForCausalLM(_config(), ResKVKernelConfig()).eval()
    model.load_state_dict(stock.state_dict())
    ids = torch.randint(5, 300, (2, 24), generator=torch.Generator().manual_seed(1))
    mask = torch.ones_like(ids)
    with torch.no_grad():
        want = stock.generate(ids, attention_mask=mask, max_new_tokens=40, do_sample=False, pad_token_id=0)
        got = model.generate(ids, attention_mask=mask, max_new_tokens=40, do_sample=False, pad_token_id=0)
    assert torch.equal(got, want)  # 24 + 40 tokens stay inside the 96-slot ring


def test_forward_returns_a_resKV_cache_and_counts_tokens():
    model = ResKVForCausalLM(_config(), ResKVKernelConfig()).eval()
    ids = torch.randint(5, 300, (1, 10))
    with torch.no_grad():
        out = model(ids)
        cache = out.past_key_values
        assert isinstance(cache, ResKVCache) and cache.get_seq_length() == 10
        out = model(ids[:, :1], past_key_values=cache)
    assert cache.get_seq_length() == 11 and all(layer.live == 11 for layer in cache.layers)
    assert out.logits.shape == (1, 1, 300)


def test_settings_are_stored_in_the_model_config():
    cfg = _config()
    model = ResKVForCausalLM(cfg, ResKVKernelConfig(sparsity=0.75, num_clusters=16))
    assert cfg.reskv_kernel_config["sparsity"] == 0.75 and model.kernel_config.num_clusters == 16
    again = ResKVForCausalLM(cfg)  # read back from the config
    assert again.kernel_config == model.kernel_config


@pytest.mark.parametrize("kw,match", [
    (dict(hidden_size=256, num_attention_heads=4, num_key_value_heads=1), "head_dim"),
    (dict(num_attention_heads=4, num_key_value_heads=2), "GQA"),
    (dict(num_attention_heads=4, num_key_value_heads=3), "multiple"),
])
def test_unsupported_shapes_rejected(kw, match):
    with pytest.raises(ValueError, match=match):
        ResKVForCausalLM(_config(**kw))


def test_forward_checks():
    model = ResKVForCausalLM(_config(), ResKVKernelConfig())
    ids = torch.randint(5, 300, (2, 6))
    with pytest.raises(ValueError, match="eval"):
        model(ids)  # training mode
    model.eval()
    with torch.no_grad():
        with pytest.raises(ValueError, match="unpadded"):
            model(ids, attention_mask=torch.tensor([[1] * 6, [0] + [1] * 5]))
        with pytest.raises(ValueError, match="ResKVCache"):
            model(ids, past_key_values=object())
        with pytest.raises(ValueError, match="contiguous"):
            model(ids, position_ids=torch.arange(1, 7)[None])
        with pytest.raises(ValueError, match="exactly one"):
            model()
        cache = model(ids).past_key_values
        with pytest.raises(ValueError, match="single-token"):
            model(ids[:, :2], past_key_values=cache)


@pytest.mark.parametrize("field", ["position_ids", "cache_position"])
@pytest.mark.parametrize("phase", ["prefill", "decode"])
def test_noncontiguous_positions_are_rejected(field, phase):
    """Positions that skip one, given either way and in either phase, are
    rejected (reskv tests/test_model.py:70-86)."""
    model = ResKVForCausalLM(_config(), ResKVKernelConfig()).eval()
    x = torch.randint(5, 300, (1, 16), generator=torch.Generator().manual_seed(2))
    cache, start = None, 0
    with torch.no_grad():
        if phase == "decode":
            cache = model(x).past_key_values
            start = x.shape[-1]
            x = x[:, :1]
        positions = torch.arange(start, start + x.shape[-1]) + 1
        if field == "position_ids":
            positions = positions.unsqueeze(0)
        with pytest.raises(ValueError, match="contiguous"):
            model(x, past_key_values=cache, **{field: positions})


def test_decode_padding_is_rejected():
    """A decode step whose mask pads the history is rejected (reskv tests/test_model.py:89-97)."""
    model = ResKVForCausalLM(_config(), ResKVKernelConfig()).eval()
    x = torch.randint(5, 300, (1, 16), generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        cache = model(x).past_key_values
        mask = torch.ones(1, 17, dtype=torch.long)
        mask[:, 0] = 0
        with pytest.raises(ValueError, match="unpadded"):
            model(x[:, :1], past_key_values=cache, attention_mask=mask)


def test_full_and_indexed_logits_keep_transformers_semantics():
    """logits_to_keep: the default keeps the last position, 0 keeps all and a
    tensor keeps the positions it names (reskv tests/test_model.py:100-109)."""
    torch.manual_seed(4)
    model = ResKVForCausalLM(_config(), ResKVKernelConfig()).eval()
    x = torch.randint(5, 300, (1, 20), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        last = model(x).logits
        full = model(x, logits_to_keep=0).logits
        selected = model(x, logits_to_keep=torch.tensor([0, 19])).logits
    assert last.shape == (1, 1, 300) and full.shape == (1, 20, 300) and selected.shape == (1, 2, 300)
    torch.testing.assert_close(last, full[:, -1:])
    torch.testing.assert_close(selected, full[:, [0, 19]])


def _small():
    return LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=1, num_attention_heads=2,
                       num_key_value_heads=2, vocab_size=32)


def test_kernel_config_round_trips_through_checkpoint(tmp_path):
    """Settings stored in the model config build the model and survive
    save/reload (reskv tests/test_config.py:148-174)."""
    settings = ResKVKernelConfig(sparsity=0.75, bits=4, num_clusters=4, max_clusters=8, rope_mode="theta")
    config = _small()
    config.reskv_kernel_config = settings.to_dict()
    model = ResKVForCausalLM(config).eval()
    assert model.kernel_config == settings
    model.save_pretrained(tmp_path)
    assert ResKVForCausalLM.from_pretrained(tmp_path).kernel_config == settings


def test_model_rejects_configuration_of_another_kind():
    """A kernel_config of another type is a TypeError; stored settings that are
    not this class's are not silently reinterpreted; an explicit configuration
    still reuses the checkpoint (reskv tests/test_config.py:177-205)."""
    config = _small()
    with pytest.raises(TypeError, match="expected ResKVKernelConfig"):
        ResKVForCausalLM(config, kernel_config={"sparsity": 0.5})
    config.reskv_kernel_config = {"sparsity": 0.5, "bits": 16, "residual_mode": "topk"}  # another method's fields
    with pytest.raises(ValueError, match="checkpoint compression settings"):
        ResKVForCausalLM(config)
    model = ResKVForCausalLM(config, kernel_config=ResKVKernelConfig())
    assert model.kernel_config == ResKVKernelConfig()


@pytest.mark.parametrize("stored", [False, 0, "", []])
def test_invalid_stored_settings_are_not_replaced_with_defaults(stored):
    """(reskv tests/test_config.py:234-241)"""
    config = _small()
    config.reskv_kernel_config = stored
    with pytest.raises(ValueError, match="checkpoint compression settings"):
        ResKVForCausalLM(config)


def test_model_rejects_configuration_of_another_architecture():
    """(reskv tests/test_config.py:214-224)"""
    from transformers import Qwen3Config

    with pytest.raises(ValueError, match="configuration"):
        ResKVForCausalLM(Qwen3Config())


def test_public_functions_survive_model_import_order():
    """Importing the model (which imports the attention module) does not shadow
    the public callables (reskv tests/test_config.py:244-255)."""
    import subprocess
    import sys

    subprocess.run([sys.executable, "-c", "from reskv_amd import ResKVForCausalLM; "
                    "from reskv_amd import attention, compress; assert callable(attention) and callable(compress)"],
                   check=True, timeout=300)


def test_from_pretrained_takes_the_kernel_config(tmp_path):
    """transformers 5 reserves ``kernel_config`` in from_pretrained; the ResKV settings still arrive."""
    LlamaForCausalLM(_config()).save_pretrained(tmp_path)
    cfg = ResKVKernelConfig(sparsity=0.5, num_clusters=16)
    model = ResKVForCausalLM.from_pretrained(tmp_path, kernel_config=cfg)
    assert model.kernel_config == cfg
    again = ResKVForCausalLM.from_pretrained(tmp_path)  # defaults when the checkpoint stores none
    assert again.kernel_config == ResKVKernelConfig()
    model.save_pretrained(tmp_path / "saved")
    reloaded = ResKVForCausalLM.from_pretrained(tmp_path / "saved")  # settings stored with the checkpoint
    assert reloaded.kernel_config == cfg


def test_half_keeps_the_rotary_frequencies_in_fp32(tmp_path):
    """``.half()`` casts every buffer; the rotary inverse frequencies stay fp32
    (equal to those of a reload with dtype=float16), so the prompt pass and the
    compressed decode rotate with the same angles and reloaded logits agree."""
    import torch

    model = ResKVForCausalLM(_config()).half().eval()
    rotary = model.model.rotary_emb
    assert rotary.inv_freq.dtype == torch.float32
    assert model.model.layers[0].mlp.gate_proj.weight.dtype == torch.float16
    model.save_pretrained(tmp_path)
    again = ResKVForCausalLM.from_pretrained(tmp_path, dtype=torch.float16)
    assert torch.equal(again.model.rotary_emb.inv_freq, rotary.inv_freq)
    assert torch.equal(model._model_frequencies(), rotary.inv_freq)
