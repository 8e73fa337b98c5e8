"""Greedy one-token decode steps replayed from a captured HIP graph.

A decode step of a model whose attention reads a ``DartHFCache`` through the
fused adapter launches the same kernels with the same arguments every step
once the cache keeps its held-tail length on the device
(``DartHFCache.enable_graph_decode``): the append writes at the device count,
the decode kernels read it there.  ``GraphDecodeStep`` captures such a step
(forward, argmax, position update) once and replays it; a step whose append
would seal a page runs eagerly (the page is quantized and the descriptor
table rebuilt), and the next step captures the graph again.  Capturing runs
the host-side bookkeeping of one step, so replays after the first call
``DartHFCache.advance_graph_step`` for theirs.

This has no counterpart in the reference, whose decode loop runs eagerly
(reference src/dart/integrations/qwen3.py:37-103 per step).
"""

from __future__ import annotations

from typing import Optional

import torch

from .huggingface import DartHFCache


class GraphDecodeStep:
    """Greedy decode steps over ``cache``: ``input_ids`` [B, 1] and ``position_ids`` [1, 1] (device int64)
    are read and advanced in place; ``logits`` holds the last step's [B, vocab] logits."""

    def __init__(self, model: torch.nn.Module, cache: DartHFCache, input_ids: torch.Tensor,
                 position_ids: torch.Tensor, *, use_graph: bool = True) -> None:
        if input_ids.ndim != 2 or input_ids.shape[1] != 1 or input_ids.device.type != "cuda":
            raise ValueError("input_ids must be a [B, 1] device tensor")
        if position_ids.shape != (1, 1) or position_ids.device != input_ids.device:
            raise ValueError("position_ids must be a [1, 1] tensor on the input's device")
        self.model = model
        self.cache = cache
        self.input_ids = input_ids
        self.position_ids = position_ids
        self.use_graph = use_graph
        self.logits: Optional[torch.Tensor] = None
        self.captures = 0
        self.eager_steps = 0
        self.replays = 0
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        self._epoch = -1  # the cache's graph_epoch when the graph was captured
        self._fresh = True  # the decode descriptors are rebuilt by an eager step before a capture

    def _forward(self) -> None:
        out = self.model(self.input_ids, position_ids=self.position_ids, past_key_values=self.cache,
                         use_cache=True, logits_to_keep=1)
        last = out.logits[:, -1]
        if self.logits is None:
            self.logits = torch.empty_like(last)
        self.logits.copy_(last)
        self.input_ids.copy_(last.argmax(-1, keepdim=True))
        self.position_ids.add_(1)

    def step(self) -> torch.Tensor:
        """Run one decode step; returns ``input_ids`` (now the generated tokens)."""
        if self.use_graph and not self.cache.graph_decode_ready():
            # device-side tail counts for every layer the prefill created (a step object may be built
            # before the prefill); the step after enabling them runs eagerly
            if not self.cache.layers or not all(layer.is_initialized for layer in self.cache.layers):
                raise RuntimeError("GraphDecodeStep needs the prompt prefilled into every layer of the cache")
            self.cache.enable_graph_decode()
            self._fresh = True
        if self._graph is not None and self.cache.graph_epoch != self._epoch:
            self._graph, self._fresh = None, True  # batch rows moved: descriptors were rebuilt
        if not self.use_graph or self._fresh or self.cache.graph_step_seals():
            self._forward()
            self.eager_steps += 1
            self._graph = None
            self._fresh = False
        elif self._graph is None:
            graph = torch.cuda.CUDAGraph()
            # each capture gets its own memory pool, released with the previous graph
            with torch.cuda.graph(graph):
                self._forward()
            graph.replay()
            self._graph = graph
            self._epoch = self.cache.graph_epoch
            self.captures += 1
        else:
            self.cache.advance_graph_step(1)
            self._graph.replay()
            self.replays += 1
        return self.input_ids


__all__ = ["GraphDecodeStep"]
