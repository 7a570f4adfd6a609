"""Llama on the installed transformers with a ResKV cache (the reference's
``reskv.models.llama.ResKVForCausalLM`` surface, reskv/models/llama.py:78-170).

Each attention layer runs in one of three modes, chosen from its layer cache:

* **prompt** (empty cache): SDPA over the prompt's own K/V, then the cache
  takes the rotated K, pre-RoPE K and V (and compresses the older part);
* **ring** (tokens cached, nothing compressed yet): SDPA over the dense ring;
* **compressed**: ``ResKVLayerCache.attend`` -- the split-K decode over the
  compressed history with the ring joined inside the split merge.

Differences from the reference that follow from the transformers release on
this image (5.x): RoPE settings come from ``config.rope_parameters``, the
model forward takes ``position_ids`` (``cache_position`` is accepted and
checked when passed), and ``from_pretrained`` hands ``kernel_config`` to the
model through its config because transformers 5 reserves that keyword.
"""

import torch
import torch.nn.functional as F
from transformers import LlamaForCausalLM
from transformers.models.llama.modeling_llama import LlamaAttention, apply_rotary_pos_emb

from ..cache import ResKVCache
from ..config import ResKVKernelConfig, _model_settings

_ROPE_TYPES = ("default", "llama3", "linear")
_GQA_RATIOS = (1, 4, 8)


def _rope_type_and_theta(config):
    """(rope_type, theta) from a transformers 5 (``rope_parameters``) or 4 (``rope_scaling``) config."""
    params = getattr(config, "rope_parameters", None) or getattr(config, "rope_scaling", None) or {}
    return params.get("rope_type", "default"), float(params.get("rope_theta", getattr(config, "rope_theta", 1e4)))


def _model_rules(config, settings):
    head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
    q_heads, kv_heads = config.num_attention_heads, config.num_key_value_heads
    yield head_dim != 128, "ResKV requires head_dim=128"
    yield kv_heads < 1 or q_heads % kv_heads, "query heads must be a positive integer multiple of KV heads"
    yield q_heads // max(kv_heads, 1) not in _GQA_RATIOS, "ResKV supports GQA ratios 1, 4, and 8"
    yield (settings.rope_mode == "model" and _rope_type_and_theta(config)[0] not in _ROPE_TYPES,
           "this release supports static default, llama3, and linear RoPE")


def _raise_first(rules):
    for failed, message in rules:
        if failed:
            raise ValueError(message)


class ResKVAttention(LlamaAttention):
    """One Llama attention layer over a ResKV layer cache (modes in the module docstring)."""

    rope_frequencies = None  # fp32 [64] or None (theta mode), set by ResKVForCausalLM.forward

    def _project(self, hidden):
        shape = (*hidden.shape[:-1], -1, self.head_dim)
        return tuple(proj(hidden).view(shape).transpose(1, 2) for proj in (self.q_proj, self.k_proj, self.v_proj))

    def forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None, **kwargs):
        batch, length = hidden_states.shape[:2]
        q, k, v = self._project(hidden_states)
        q_rot, k_rot = apply_rotary_pos_emb(q, k, *position_embeddings)
        layer = None if past_key_values is None else past_key_values.layers[self.layer_idx]
        if layer is None or layer.length == 0:
            out = F.scaled_dot_product_attention(q_rot, k_rot, v, attn_mask=attention_mask,
                                                 is_causal=attention_mask is None and length > 1,
                                                 enable_gqa=True, scale=self.scaling)
            if layer is not None:
                layer.update(k_rot, v, {"raw_keys": k})
        else:
            if length != 1:
                raise ValueError("only single-token continuation is supported")
            ring_k, ring_v = layer.update(k_rot, v, {"raw_keys": k})
            if layer.compressed is None:
                out = F.scaled_dot_product_attention(q_rot, ring_k, ring_v, enable_gqa=True, scale=self.scaling)
            else:
                freq = self.rope_frequencies if layer.config.rope_mode == "model" else None
                out = layer.attend(q.contiguous(), q_rot.contiguous(), scaling=self.scaling, inv_freq=freq,
                                   rope_theta=_rope_type_and_theta(self.config)[1])
        out = out.transpose(1, 2).reshape(batch, length, -1)
        return self.o_proj(out), None


class ResKVForCausalLM(LlamaForCausalLM):
    """Llama with a ResKV cache: fp16 inference, 128-dimensional heads, GQA ratios
    1/4/8, equal-length unpadded batches (padded generation is rejected)."""

    def __init__(self, config, kernel_config: ResKVKernelConfig | None = None):
        if config.model_type != "llama":
            raise ValueError("ResKV inference requires a Llama configuration")
        settings = _model_settings(config, kernel_config, ResKVKernelConfig, "reskv_kernel_config")
        _raise_first(_model_rules(config, settings))
        config._attn_implementation = "sdpa"
        super().__init__(config)
        self.kernel_config = settings
        for idx, block in enumerate(self.model.layers):
            block.self_attn = ResKVAttention(config, idx)
        self._freq32 = None
        self.post_init()

    @classmethod
    def _supports_default_dynamic_cache(cls):
        return False

    @classmethod
    def from_pretrained(cls, pretrained_model_name_or_path, *args, kernel_config=None, **kwargs):
        """``from_pretrained(path, kernel_config=ResKVKernelConfig(...))``; any other
        ``kernel_config`` value goes on to transformers (its hub-kernel option)."""
        if isinstance(kernel_config, ResKVKernelConfig):
            from transformers import AutoConfig

            config = kwargs.pop("config", None) or AutoConfig.from_pretrained(pretrained_model_name_or_path)
            config.reskv_kernel_config = kernel_config.to_dict()
            kwargs["config"] = config
        elif kernel_config is not None:
            kwargs["kernel_config"] = kernel_config
        return super().from_pretrained(pretrained_model_name_or_path, *args, **kwargs)

    def _apply(self, fn, recurse=True):
        """Module moves and casts (``.half()``, ``.to()``, ``.cuda()``) keep the
        rotary inverse frequencies in fp32: rounded to fp16 they would move every
        RoPE angle of the prompt pass, away from the fp32 angles of the
        compressed decode, and a reload (which keeps them fp32) would compute
        different logits."""
        rotary = getattr(getattr(self, "model", None), "rotary_emb", None)
        keep = {}
        if rotary is not None:
            keep = {n: b for n, b in rotary._buffers.items()
                    if b is not None and "inv_freq" in n and b.dtype == torch.float32}
        out = super()._apply(fn, recurse)
        for n, b in keep.items():
            cur = rotary._buffers[n]
            if cur is not None and cur.dtype != torch.float32:
                rotary._buffers[n] = b.to(cur.device)
        return out

    def _model_frequencies(self):
        """The rotary inverse frequencies in fp32 (recomputed once if the buffer
        arrived rounded, e.g. from a checkpoint stored that way)."""
        rotary = self.model.rotary_emb
        if rotary.inv_freq.dtype == torch.float32:
            return rotary.inv_freq
        if self._freq32 is None or self._freq32.device != rotary.inv_freq.device:
            if rotary.rope_type == "default":
                fresh, _ = rotary.compute_default_rope_parameters(self.config)
            else:
                from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

                fresh, _ = ROPE_INIT_FUNCTIONS[rotary.rope_type](self.config)
            self._freq32 = fresh.float().to(rotary.inv_freq.device)
        return self._freq32

    def _check_call(self, input_ids, inputs_embeds, labels, past_key_values, attention_mask, positions):
        if (input_ids is None) == (inputs_embeds is None):
            raise ValueError("provide exactly one of input_ids or inputs_embeds")
        if labels is not None or self.training:
            raise ValueError("ResKV is an inference implementation; call model.eval()")
        if past_key_values is not None and not isinstance(past_key_values, ResKVCache):
            raise ValueError("past_key_values must be a ResKVCache")
        if attention_mask is not None and not bool(attention_mask.eq(1).all()):
            raise ValueError("ResKV requires equal-length unpadded batches")
        given = [p for p in positions if p is not None]
        if given:
            source = input_ids if input_ids is not None else inputs_embeds
            length = input_ids.shape[-1] if input_ids is not None else inputs_embeds.shape[-2]
            start = 0 if past_key_values is None else past_key_values.get_seq_length()
            want = torch.arange(start, start + length, device=source.device)
            if any(p.device != source.device or not bool(p.eq(want).all()) for p in given):
                raise ValueError("ResKV positions must be contiguous and start at zero")

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
                inputs_embeds=None, labels=None, use_cache=None, cache_position=None, logits_to_keep=1, **kwargs):
        if use_cache is None:
            use_cache = self.config.use_cache
        self._check_call(input_ids, inputs_embeds, labels, past_key_values, attention_mask,
                         (position_ids, cache_position))
        if use_cache and past_key_values is None:
            past_key_values = ResKVCache(self.kernel_config, len(self.model.layers))
        freq = self._model_frequencies() if self.kernel_config.rope_mode == "model" else None
        for block in self.model.layers:
            # a plain attribute, not a registered buffer: refreshed on every call
            object.__setattr__(block.self_attn, "rope_frequencies", freq)
        return super().forward(input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                               past_key_values=past_key_values, inputs_embeds=inputs_embeds, use_cache=use_cache,
                               logits_to_keep=logits_to_keep, **kwargs)
