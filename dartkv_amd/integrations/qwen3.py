"""Qwen3 attention adapter that decodes straight from the packed Dart pages.

Mirrors reference src/dart/integrations/qwen3.py:30-124.  Prefill (and any
call that is not a one-token decode over an existing layer) uses the model's
configured attention on the dense tensors ``DartHFCache.update`` returns; a
one-token decode calls ``fused_dart_attention`` on the layer's packed cache,
which runs the HIP split-K page kernels.

The forward accepts the cache under both keyword names Transformers has used
(``past_key_values`` in 5.x, ``past_key_value`` in 4.x).

When the cache keeps its held-tail length on the device
(``DartHFCache.enable_graph_decode``) and the token extends the tail, a
one-token decode runs one GEMM for the query, key and value projections (their
weights are views of one matrix) and one kernel for the query/key RMSNorm, the
rotary embedding and the append (``dkv_decode_prep``) before the page
attention, instead of the Transformers ops; that is about 25 fewer launches
per layer and step.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from .. import _lib
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


def _fused_qkv_weight(attn: nn.Module) -> Optional[torch.Tensor]:
    """The q/k/v projection weights as one [(Hq + 2 Hkv) D, hidden] matrix whose row blocks the three
    projections' weights are views of (so one GEMM computes all three), or None when they have biases
    or no longer share that storage."""
    w = getattr(attn, "_dart_qkv", None)
    if w is None:
        return None
    q, k, v = attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight
    nq, nk = q.shape[0], k.shape[0]
    if (q.data_ptr() != w.data_ptr() or k.data_ptr() != w[nq:].data_ptr()
            or v.data_ptr() != w[nq + nk:].data_ptr()):
        return None
    return w


def _share_qkv_storage(attn: nn.Module) -> None:
    if any(getattr(getattr(attn, n), "bias", None) is not None for n in ("q_proj", "k_proj", "v_proj")):
        return
    with torch.no_grad():
        w = torch.cat([attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight], 0).contiguous()
    nq, nk = attn.q_proj.weight.shape[0], attn.k_proj.weight.shape[0]
    attn.q_proj.weight = nn.Parameter(w[:nq], requires_grad=attn.q_proj.weight.requires_grad)
    attn.k_proj.weight = nn.Parameter(w[nq:nq + nk], requires_grad=attn.k_proj.weight.requires_grad)
    attn.v_proj.weight = nn.Parameter(w[nq + nk:], requires_grad=attn.v_proj.weight.requires_grad)
    attn._dart_qkv = w


def _prepared_decode(attn: nn.Module, hidden_states: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     cache: DartHFCache, layer_idx: int, w_qkv: torch.Tensor) -> torch.Tensor:
    """One-token decode with the fused QKV projection and the preparation kernel (RMSNorm + rotary
    embedding + append into the held tail), then the packed-page attention.  Returns [B, 1, Hq, D]."""
    layer = cache.layer_for_attention(layer_idx)
    B = hidden_states.shape[0]
    D = attn.head_dim
    Hq = attn.q_proj.weight.shape[0] // D
    Hkv = attn.k_proj.weight.shape[0] // D
    qkv = torch.nn.functional.linear(hidden_states.reshape(B, -1), w_qkv)
    q = torch.empty(B, Hq, 1, D, dtype=hidden_states.dtype, device=hidden_states.device)
    a = _lib.DecodePrepArgs()
    a.qkv, a.qkv_sb = qkv.data_ptr(), qkv.stride(0)
    a.q_weight, a.k_weight = attn.q_norm.weight.data_ptr(), attn.k_norm.weight.data_ptr()
    a.eps = float(attn.q_norm.variance_epsilon)
    a.cos, a.sin = cos.data_ptr(), sin.data_ptr()
    a.q_out = q.data_ptr()
    a.tail_key, a.tail_value = layer._tail_key.data_ptr(), layer._tail_value.data_ptr()
    a.tail_pos = layer.device_tail.data_ptr()
    a.B, a.Hq, a.Hkv, a.D = B, Hq, Hkv, D
    a.cap = layer._tail_key.shape[2]
    a.dtype = _lib.dtype_code(hidden_states.dtype)
    _lib.check(_lib.load().dkv_decode_prep(a, _lib.stream_ptr(hidden_states.device)), "dkv_decode_prep")
    cache.commit_prepared_append(layer_idx)
    return fused_dart_attention(q, layer, scale=attn.scaling, fallback=True).transpose(1, 2)


def _can_prepare(attn: nn.Module, hidden_states: torch.Tensor, cos: torch.Tensor, cache, layer_idx: int,
                 kwargs: dict) -> Optional[torch.Tensor]:
    if not isinstance(cache, DartHFCache) or hidden_states.shape[1] != 1 or kwargs.get("output_attentions"):
        return None
    if hidden_states.dtype not in (torch.bfloat16, torch.float16) or attn.head_dim != 128:
        return None
    if cos.dtype != hidden_states.dtype or cos.shape[0] != 1 or cos.numel() != attn.head_dim or not cos.is_contiguous():
        return None
    if attn.q_norm.weight.dtype != hidden_states.dtype or attn.k_norm.weight.dtype != hidden_states.dtype:
        return None
    if not cache.prepared_append_ok(layer_idx):
        return None
    return _fused_qkv_weight(attn)


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
            cos, sin = position_embeddings
            w_qkv = _can_prepare(self, hidden_states, cos, cache, self.layer_idx, kwargs)
            if w_qkv is not None and sin.is_contiguous():
                attn_output = _prepared_decode(self, hidden_states, cos, sin, cache, self.layer_idx, w_qkv)
                attn_output = attn_output.reshape(*input_shape, -1).contiguous()
                return self.o_proj(attn_output), None
            hidden_shape = (*input_shape, -1, self.head_dim)
            query_states = self.q_norm(self.q_proj(hidden_states).view(hidden_shape)).transpose(1, 2)
            key_states = self.k_norm(self.k_proj(hidden_states).view(hidden_shape)).transpose(1, 2)
            value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)

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
        _share_qkv_storage(replacement)
        layer.self_attn = replacement
    return model


__all__ = ["attach_dart_fused_attention", "build_dart_qwen3_attention_class"]
