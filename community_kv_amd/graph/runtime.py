"""Prefill partition hand-off (reference: community_kv/graph/runtime.py:29-176).

The reference runs Leiden on worker threads, one job per layer.  Here a job
runs ``build_partitioned_layer`` (top-k graph, native batched Leiden, state
build) synchronously on the submitting stream after the completion event, so
no extra threads or streams are created.  A *label provider*, a callable
``provider(layer_idx, keys, topk_indices, topk_scores) -> community_ids
[graphs, S]``, may replace Leiden; its labels are turned into decode state by
``build_layer_from_labels`` with the modularity state of the top-k edges.
"""

from __future__ import annotations

from typing import Any, Callable

import torch

from community_kv_amd.config import CommunityKVConfig, GraphAggregation, PartitionConfig
from community_kv_amd.graph.kernels.state_build import TopkEdges
from community_kv_amd.graph.partition import (PartitionedLayer, build_adjacency, build_layer_from_labels,
                                              build_partitioned_layer)


class PartitionRuntime:
    def __init__(self, *, algorithm: CommunityKVConfig, scheduling: PartitionConfig, max_layers: int,
                 label_provider: Callable[..., torch.Tensor] | None = None) -> None:
        if max_layers <= 0:
            raise ValueError("max_layers must be positive")
        self.algorithm = algorithm
        self.scheduling = scheduling
        self.max_layers = max_layers
        self.label_provider = label_provider
        self._results: dict[int, PartitionedLayer] = {}

    def reset(self) -> None:
        self._results.clear()

    def submit(self, *, layer_idx: int, topk_indices: torch.Tensor, topk_scores: torch.Tensor, keys: torch.Tensor,
               completion_event: Any, resolution: float, max_decode_tokens: int) -> None:
        if layer_idx in self._results:
            raise ValueError(f"layer {layer_idx} was already submitted")
        if not 0 <= layer_idx < self.max_layers:
            raise ValueError("layer index out of range")
        if completion_event is not None and hasattr(completion_event, "synchronize"):
            completion_event.synchronize()
        cfg = self.algorithm
        aggregation = GraphAggregation(cfg.aggregation)
        if self.label_provider is None:
            self._results[layer_idx] = build_partitioned_layer(
                layer_idx=layer_idx, topk_indices=topk_indices, topk_scores=topk_scores, keys=keys,
                num_sink=cfg.num_sink, lam=cfg.lam, leiden_resolution=resolution, leiden_seed=cfg.leiden_seed,
                max_decode_tokens=max_decode_tokens, aggregation=aggregation)
            return
        labels = self.label_provider(layer_idx, keys, topk_indices, topk_scores)
        edges = topk_edges = None
        if topk_indices is not None and topk_indices.numel():
            seq_len = keys.shape[1]
            heads, rows, kappa = topk_indices.shape
            graphs = labels.shape[0]
            group = heads // graphs
            row0 = kappa - 1 + cfg.num_sink
            if keys.device.type == "cuda":
                # the device state build takes the top-k edges as they are (no
                # edge list to build, sort and coalesce: Leiden is not run here)
                topk_edges = TopkEdges(indices=topk_indices, scores=topk_scores, row0=row0, group=group,
                                       lam=cfg.lam)
            else:
                base = torch.arange(row0, row0 + rows, device=topk_indices.device)
                idx = topk_indices.reshape(graphs, group * rows, kappa)
                sc = topk_scores.reshape(graphs, group * rows, kappa)
                pos = base.repeat(group).unsqueeze(0).expand(graphs, -1)
                edges = build_adjacency(idx, sc, pos, seq_len=seq_len, lam=cfg.lam)
        self._results[layer_idx] = build_layer_from_labels(
            layer_idx=layer_idx, community_ids=labels, keys=keys, num_sink=cfg.num_sink,
            max_decode_tokens=max_decode_tokens, query_heads=topk_indices.shape[0], aggregation=aggregation,
            edges=edges, topk_edges=topk_edges)

    def wait(self, callback: Callable[[PartitionedLayer], Any]) -> None:
        for idx in sorted(self._results):
            callback(self._results[idx])
        self._results.clear()

    def shutdown(self) -> None:
        self._results.clear()


__all__ = ["PartitionRuntime"]
