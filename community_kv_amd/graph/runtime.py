"""Prefill partition hand-off (reference: community_kv/graph/runtime.py:29-176).

The reference runs Leiden on worker threads, one job per layer, each job on
its own stream after the layer's completion event.  Here a job runs
``build_partitioned_layer`` (top-k graph, native batched Leiden, state build)
the same way on the model's GPU: ``PartitionConfig.workers_per_device`` worker
threads (jobs of different layers run concurrently), a stream of default priority
per job that waits on the completion event, the stream synchronised before the
result is handed over, so the partition of layer i overlaps the prefill of
layers i+1, ...; with ``PartitionConfig(overlap=False)`` jobs run inline on the
submitting stream.  A *label provider*, a callable
``provider(layer_idx, keys, topk_indices, topk_scores) -> community_ids
[graphs, S]``, may replace Leiden; its labels are turned into decode state by
``build_layer_from_labels`` with the modularity state of the top-k edges.
"""

from __future__ import annotations

import dataclasses
from concurrent.futures import Future, ThreadPoolExecutor
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
        self._futures: dict[int, Future] = {}
        self._executor: ThreadPoolExecutor | None = None

    def reset(self) -> None:
        """Drops every pending and finished job.  Waits for the running ones;
        the first job error is raised once, after the runtime is empty again,
        so a later request starts clean."""
        futures = list(self._futures.values())
        self._futures.clear()
        self._results.clear()
        error = None
        for future in futures:
            exc = future.exception()
            if exc is not None and error is None:
                error = exc
        if error is not None:
            raise error

    def _pool(self) -> ThreadPoolExecutor:
        if self._executor is None:
            workers = max(1, min(self.max_layers, self.scheduling.workers_per_device))
            self._executor = ThreadPoolExecutor(max_workers=workers, thread_name_prefix="ckv-partition")
        return self._executor

    def _run_job(self, *, layer_idx: int, topk_indices: torch.Tensor, topk_scores: torch.Tensor,
                 keys: torch.Tensor, completion_event: Any, resolution: float,
                 max_decode_tokens: int) -> PartitionedLayer:
        cfg = self.algorithm
        with torch.cuda.device(keys.device):
            stream = torch.cuda.Stream(device=keys.device)
            if completion_event is not None:
                stream.wait_event(completion_event)
            with torch.cuda.stream(stream):
                layer = build_partitioned_layer(
                    layer_idx=layer_idx, topk_indices=topk_indices, topk_scores=topk_scores, keys=keys,
                    num_sink=cfg.num_sink, lam=cfg.lam, leiden_resolution=resolution, leiden_seed=cfg.leiden_seed,
                    max_decode_tokens=max_decode_tokens, aggregation=GraphAggregation(cfg.aggregation))
            stream.synchronize()
        return layer

    def submit(self, *, layer_idx: int, topk_indices: torch.Tensor, topk_scores: torch.Tensor, keys: torch.Tensor,
               completion_event: Any, resolution: float, max_decode_tokens: int) -> None:
        if layer_idx in self._results or layer_idx in self._futures:
            raise ValueError(f"layer {layer_idx} was already submitted")
        if not 0 <= layer_idx < self.max_layers:
            raise ValueError("layer index out of range")
        if not all(_same_device(d, keys.device) for d in self.scheduling.devices):
            raise NotImplementedError("partition offload to another GPU is not part of this build")
        if self.label_provider is None and self.scheduling.overlap and keys.device.type == "cuda":
            self._futures[layer_idx] = self._pool().submit(
                self._run_job, layer_idx=layer_idx, topk_indices=topk_indices, topk_scores=topk_scores, keys=keys,
                completion_event=completion_event, resolution=resolution, max_decode_tokens=max_decode_tokens)
            return
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
        for idx, future in sorted(self._futures.items()):
            layer = future.result()
            # made on the job's stream, used from now on by the current one
            consumer = torch.cuda.current_stream(layer.centroids.device)
            for value in vars_of(layer):
                if isinstance(value, torch.Tensor) and value.is_cuda:
                    value.record_stream(consumer)
            self._results[idx] = layer
        self._futures.clear()
        for idx in sorted(self._results):
            callback(self._results[idx])
        self._results.clear()

    def shutdown(self) -> None:
        self.reset()
        if self._executor is not None:
            self._executor.shutdown(wait=True)
            self._executor = None


def _same_device(name: Any, device: torch.device) -> bool:
    """Whether the configured device `name` is `device`; a CUDA device
    without an index means the current one."""
    d = torch.device(name)
    if d.type != device.type:
        return False
    if d.type == "cuda":
        current = torch.cuda.current_device() if torch.cuda.is_available() else 0
        return (current if d.index is None else d.index) == (current if device.index is None else device.index)
    return True


def vars_of(layer: PartitionedLayer) -> list[Any]:
    return [getattr(layer, f.name) for f in dataclasses.fields(layer)]


__all__ = ["PartitionRuntime"]
