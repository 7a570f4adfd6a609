"""Llama model patch for the installed transformers (reskv/models/llama.py:1-170).

``ResKVForCausalLM`` is a ``LlamaForCausalLM`` whose attention layers keep
their keys and values in a ``ResKVCache``.  The prompt attends densely (SDPA)
and is then compressed by the gfx950 kernels.  Each later token attends over
the compressed history plus the dense ring of recent tokens through
``ResKVLayerCache.attend`` (split-K decode kernel, exact merge with the ring);
before the first group is compressed it attends densely over the ring.

Differences from the reference that follow from the transformers release on
this image (5.x): RoPE settings come from ``config.rope_parameters`` and the
model forward takes ``position_ids`` (``cache_position`` is accepted and
checked when a caller passes it).
"""

import torch
import torch.nn.functional as F
from transformers import LlamaForCausalLM
from transformers.models.llama.modeling_llama import LlamaAttention, LlamaMLP, apply_rotary_pos_emb

from ..cache import ResKVCache
from ..config import ResKVKernelConfig, _model_settings

_ROPE_TYPES = ("default", "llama3", "linear")


def _rope_parameters(config):
    """(rope_type, theta) from a transformers 5 (``rope_parameters``) or 4 (``rope_scaling``) config."""
    params = getattr(config, "rope_parameters", None) or getattr(config, "rope_scaling", None) or {}
    theta = params.get("rope_theta", getattr(config, "rope_theta", 10000.0))
    return params.get("rope_type", "default"), float(theta)


class ResKVMLP(LlamaMLP):
    """Gated MLP for inference: the up projection multiplies the activated gate in place."""

    def forward(self, hidden_states):
        if self.training or torch.is_grad_enabled():
            return super().forward(hidden_states)
        gate = self.act_fn(self.gate_proj(hidden_states))
        gate.mul_(self.up_proj(hidden_states))
        return self.down_proj(gate)


class ResKVAttention(LlamaAttention):
    """Attention over the compressed history and the dense ring (reskv/models/llama.py:25-75)."""

    rope_frequencies = None  # fp32 [64], set by ResKVForCausalLM.forward

    def forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                **kwargs):
        shape = hidden_states.shape[:-1]
        heads = (*shape, -1, self.head_dim)
        q = self.q_proj(hidden_states).view(heads).transpose(1, 2)
        k = self.k_proj(hidden_states).view(heads).transpose(1, 2)
        v = self.v_proj(hidden_states).view(heads).transpose(1, 2)
        cos, sin = position_embeddings
        qr, kr = apply_rotary_pos_emb(q, k, cos, sin)
        layer = None if past_key_values is None else past_key_values.layers[self.layer_idx]
        if layer is not None and layer.length > 0:
            if shape[1] != 1:
                raise ValueError("only single-token continuation is supported")
            ring_k, ring_v = layer.update(kr, v, {"raw_keys": k})
            if layer.compressed is not None:
                model_freq = layer.config.rope_mode == "model"
                out = layer.attend(q.contiguous(), qr.contiguous(), scaling=self.scaling,
                                   inv_freq=self.rope_frequencies if model_freq else None,
                                   rope_theta=_rope_parameters(self.config)[1])
            else:
                out = F.scaled_dot_product_attention(qr, ring_k, ring_v, enable_gqa=True, scale=self.scaling)
        else:
            # the prompt attends to its dense K/V; the cache compresses afterwards
            out = F.scaled_dot_product_attention(qr, kr, v, attn_mask=attention_mask,
                                                 is_causal=attention_mask is None and shape[1] > 1,
                                                 enable_gqa=True, scale=self.scaling)
            if layer is not None:
                layer.update(kr, v, {"raw_keys": k})
        out = out.transpose(1, 2).reshape(*shape, -1).contiguous()
        return self.o_proj(out), None


class ResKVForCausalLM(LlamaForCausalLM):
    """Llama with a ResKV cache (reskv/models/llama.py:78-170).

    fp16 inference with 128-dimensional heads, GQA ratios 1/4/8 and equal-length
    unpadded batches; padded generation is rejected.
    """

    def __init__(self, config, kernel_config: ResKVKernelConfig | None = None):
        if config.model_type != "llama":
            raise ValueError("ResKV inference requires a Llama configuration")
        settings = _model_settings(config, kernel_config, ResKVKernelConfig, "reskv_kernel_config")
        if (getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads) != 128:
            raise ValueError("ResKV requires head_dim=128")
        if config.num_key_value_heads < 1 or config.num_attention_heads % config.num_key_value_heads:
            raise ValueError("query heads must be a positive integer multiple of KV heads")
        if config.num_attention_heads // config.num_key_value_heads not in (1, 4, 8):
            raise ValueError("ResKV supports GQA ratios 1, 4, and 8")
        if settings.rope_mode == "model" and _rope_parameters(config)[0] not in _ROPE_TYPES:
            raise ValueError("this release supports static default, llama3, and linear RoPE")
        config._attn_implementation = "sdpa"
        super().__init__(config)
        self.kernel_config = settings
        for idx, layer in enumerate(self.model.layers):
            layer.self_attn = ResKVAttention(config, idx)
            layer.mlp = ResKVMLP(config)
        self._fp32_freq = None
        self.post_init()

    @classmethod
    def _supports_default_dynamic_cache(cls):
        return False

    @classmethod
    def from_pretrained(cls, pretrained_model_name_or_path, *args, kernel_config=None, **kwargs):
        """``from_pretrained(path, kernel_config=ResKVKernelConfig(...))`` as in the reference.

        transformers 5 reserves the ``kernel_config`` keyword for its hub
        kernels; a ResKV configuration is handed over through the model config
        (``reskv_kernel_config``, which ``__init__`` reads), any other value
        goes on to transformers."""
        if isinstance(kernel_config, ResKVKernelConfig):
            from transformers import AutoConfig

            config = kwargs.pop("config", None)
            if config is None:
                config = AutoConfig.from_pretrained(pretrained_model_name_or_path)
            config.reskv_kernel_config = kernel_config.to_dict()
            kwargs["config"] = config
        elif kernel_config is not None:
            kwargs["kernel_config"] = kernel_config
        return super().from_pretrained(pretrained_model_name_or_path, *args, **kwargs)

    def _frequencies(self):
        """The model's RoPE inverse frequencies in fp32 (recomputed when ``.half()`` cast the buffer)."""
        rotary = self.model.rotary_emb
        freq = rotary.inv_freq
        if freq.dtype == torch.float32:
            return freq
        if self._fp32_freq is None or self._fp32_freq.device != freq.device:
            if rotary.rope_type == "default":
                fresh, _ = rotary.compute_default_rope_parameters(self.config)
            else:
                from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

                fresh, _ = ROPE_INIT_FUNCTIONS[rotary.rope_type](self.config)
            self._fp32_freq = fresh.float().to(freq.device)
        return self._fp32_freq

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
                inputs_embeds=None, labels=None, use_cache=None, cache_position=None, logits_to_keep=1, **kwargs):
        use_cache = self.config.use_cache if use_cache is None else use_cache
        if (input_ids is None) == (inputs_embeds is None):
            raise ValueError("provide exactly one of input_ids or inputs_embeds")
        if labels is not None or self.training:
            raise ValueError("ResKV is an inference implementation; call model.eval()")
        if past_key_values is not None and not isinstance(past_key_values, ResKVCache):
            raise ValueError("past_key_values must be a ResKVCache")
        if use_cache and past_key_values is None:
            past_key_values = ResKVCache(self.kernel_config, len(self.model.layers))
        if attention_mask is not None and not bool(attention_mask.eq(1).all()):
            raise ValueError("ResKV requires equal-length unpadded batches")
        if position_ids is not None or cache_position is not None:
            length = input_ids.shape[-1] if input_ids is not None else inputs_embeds.shape[-2]
            device = input_ids.device if input_ids is not None else inputs_embeds.device
            seen = 0 if past_key_values is None else past_key_values.get_seq_length()
            expected = torch.arange(seen, seen + length, device=device)
            for positions in (position_ids, cache_position):
                if positions is not None and (positions.device != device or not bool(positions.eq(expected).all())):
                    raise ValueError("ResKV positions must be contiguous and start at zero")
        freq = self._frequencies() if self.kernel_config.rope_mode == "model" else None
        for layer in self.model.layers:
            # a plain attribute, not a registered buffer: refreshed every call
            object.__setattr__(layer.self_attn, "rope_frequencies", freq)
        return super().forward(input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                               past_key_values=past_key_values, inputs_embeds=inputs_embeds, use_cache=use_cache,
                               logits_to_keep=logits_to_keep, **kwargs)
