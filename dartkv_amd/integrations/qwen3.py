"""Qwen3 attention adapter that decodes straight from the packed Dart pages.

Mirrors reference src/dart/integrations/qwen3.py:30-124.  Prefill (and any
call that is not a one-token decode over an existing layer) uses the model's
configured attention on the dense tensors ``DartHFCache.update`` returns; a
one-token decode calls ``fused_dart_attention`` on the layer's packed cache,
which runs the HIP split-K page kernels.

The forward accepts the cache under both keyword names Transformers has used
(``past_key_values`` in 5.x, ``past_key_value`` in 4.x).
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from ..fused_attention import fused_dart_attention
from .huggingface import DartHFCache


def _qwen3_modules():
    from transformers.models.qwen3 import modeling_qwen3 as modules

    return modules


def _attention_interface(modules, config):
    implementation = config._attn_implementation
    functions = modules.ALL_ATTENTION_FUNCTIONS
    if implementation in (None, "eager"):
        return modules.eager_attention_forward
    if hasattr(functions, "get_interface"):
        return functions.get_interface(implementation, modules.eager_attention_forward)
    return functions[implementation]


class DartQwen3Attention:  # replaced by build_dart_qwen3_attention_class()
    """Placeholder; the real class subclasses the installed Qwen3Attention."""


def build_dart_qwen3_attention_class():
    """Build the Qwen3 attention subclass against the installed Transformers."""
    modules = _qwen3_modules()
    base_attention = modules.Qwen3Attention

    class _DartQwen3Attention(base_attention):
        def forward(
            self,
            hidden_states: torch.Tensor,
            position_embeddings: tuple[torch.Tensor, torch.Tensor] = None,
            attention_mask: Optional[torch.Tensor] = None,
            past_key_values=None,
            cache_position: Optional[torch.LongTensor] = None,
            past_key_value=None,
            **kwargs,
        ):
            cache = past_key_values if past_key_values is not None else past_key_value
            input_shape = hidden_states.shape[:-1]
            hidden_shape = (*input_shape, -1, self.head_dim)
            query_states = self.q_norm(self.q_proj(hidden_states).view(hidden_shape)).transpose(1, 2)
            key_states = self.k_norm(self.k_proj(hidden_states).view(hidden_shape)).transpose(1, 2)
            value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)

            cos, sin = position_embeddings
            query_states, key_states = modules.apply_rotary_pos_emb(query_states, key_states, cos, sin)

            use_dart_decode = isinstance(cache, DartHFCache)
            if cache is not None:
                cache_kwargs = {"sin": sin, "cos": cos, "cache_position": cache_position}
                if use_dart_decode:
                    cache_kwargs["dart_fused_attention"] = True
                key_states, value_states = cache.update(key_states, value_states, self.layer_idx, cache_kwargs)

            output_attentions = bool(kwargs.get("output_attentions", False))
            if (use_dart_decode and not cache.last_update_was_prefill(self.layer_idx)
                    and query_states.shape[-2] == 1 and not output_attentions):
                attn_output = fused_dart_attention(
                    query_states, cache.layer_for_attention(self.layer_idx), scale=self.scaling, fallback=True,
                ).transpose(1, 2)
                attn_weights = None
            else:
                attention_interface = _attention_interface(modules, self.config)
                attn_output, attn_weights = attention_interface(
                    self,
                    query_states,
                    key_states,
                    value_states,
                    attention_mask,
                    dropout=0.0 if not self.training else self.attention_dropout,
                    scaling=self.scaling,
                    sliding_window=self.sliding_window,
                    **kwargs,
                )

            attn_output = attn_output.reshape(*input_shape, -1).contiguous()
            attn_output = self.o_proj(attn_output)
            return attn_output, attn_weights

    _DartQwen3Attention.__name__ = "DartQwen3Attention"
    _DartQwen3Attention.__qualname__ = "DartQwen3Attention"
    return _DartQwen3Attention


def attach_dart_fused_attention(model: nn.Module) -> nn.Module:
    """Replace every Qwen3 self-attention module with the Dart adapter."""
    attention_class = build_dart_qwen3_attention_class()
    layers = getattr(getattr(model, "model", None), "layers", None)
    if layers is None:
        raise TypeError("attach_dart_fused_attention expects a Qwen3 causal-LM model")
    for layer_idx, layer in enumerate(layers):
        original = layer.self_attn
        reference_parameter = next(original.parameters())
        with torch.device(reference_parameter.device):
            replacement = attention_class(model.config, layer_idx)
        replacement.to(dtype=reference_parameter.dtype)
        replacement.load_state_dict(original.state_dict())
        replacement.train(original.training)
        layer.self_attn = replacement
    return model


__all__ = ["attach_dart_fused_attention", "build_dart_qwen3_attention_class"]
