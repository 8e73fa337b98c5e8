"""Integrations with external model libraries (reference src/dart/integrations/__init__.py)."""

from .graph import GraphDecodeStep
from .huggingface import DartCacheLayer, DartHFCache
from .qwen3 import attach_dart_fused_attention, build_dart_qwen3_attention_class

__all__ = ["DartCacheLayer", "DartHFCache", "GraphDecodeStep", "attach_dart_fused_attention",
           "build_dart_qwen3_attention_class"]
