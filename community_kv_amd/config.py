"""Request configuration (reference: community_kv/config.py:9-70).

``GraphAggregation``, ``CommunityKVConfig`` and ``PartitionConfig`` keep the
reference's names, fields, defaults and validation.  ``CommunityKVConfig``
adds four options of this build, all defaulting to the reference behaviour:

* ``local_window``: number of most recent tokens before the current one that
  are always attended (set union with the selected communities).
* ``selection``: ``"budget"`` (reference weighted threshold selection) or
  ``"topk"`` (the ``topk_communities`` best communities, taken whole, capped at
  ``max_selected`` tokens).
* ``assignment``: ``"delta_q"`` (reference modularity-gain rule) or
  ``"nearest_centroid"`` (join the nearest centroid, running-mean update).
* ``include_current``: attend the current token (reference: always).
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum


class GraphAggregation(str, Enum):
    """How query-head top-k edges are combined into layer graphs."""

    PER_QUERY_HEAD = "per_query_head"
    QUERY_GROUP = "query_group"
    LAYER_WISE = "layer_wise"

    def graph_count(self, *, query_heads: int, kv_heads: int) -> int:
        if query_heads <= 0 or kv_heads <= 0 or query_heads % kv_heads:
            raise ValueError("query heads must divide evenly into KV-head groups")
        if self is GraphAggregation.PER_QUERY_HEAD:
            return query_heads
        if self is GraphAggregation.QUERY_GROUP:
            return kv_heads
        return 1

    def retrieval_head_count(self, *, query_heads: int, kv_heads: int) -> int:
        return max(self.graph_count(query_heads=query_heads, kv_heads=kv_heads), kv_heads)


SELECTION_MODES = ("budget", "topk")
ASSIGNMENT_MODES = ("delta_q", "nearest_centroid")


@dataclass(frozen=True, slots=True)
class CommunityKVConfig:
    """Configuration whose values are fixed for one captured request."""

    token_budget: int = 4096
    num_sink: int = 10
    lam: float = 0.5
    aggregation: GraphAggregation = GraphAggregation.PER_QUERY_HEAD
    leiden_resolution: float = 1.0
    leiden_seed: int = 0
    local_window: int = 0
    selection: str = "budget"
    topk_communities: int = 8
    max_selected: int = 0
    assignment: str = "delta_q"
    include_current: bool = True

    def __post_init__(self) -> None:
        if isinstance(self.aggregation, str):
            object.__setattr__(self, "aggregation", GraphAggregation(self.aggregation))
        if self.token_budget <= 0 or self.token_budget % 64:
            raise ValueError("token_budget must be a positive multiple of 64")
        if self.num_sink < 0 or self.num_sink + 1 >= self.token_budget:
            raise ValueError("num_sink leaves no selected-token capacity")
        if not 0.0 <= self.lam <= 1.0:
            raise ValueError("lam must be in [0, 1]")
        if self.leiden_resolution <= 0:
            raise ValueError("leiden_resolution must be positive")
        if self.local_window < 0:
            raise ValueError("local_window must be non-negative")
        if self.selection not in SELECTION_MODES:
            raise ValueError(f"selection must be one of {SELECTION_MODES}")
        if self.selection == "topk" and (self.topk_communities <= 0 or self.max_selected <= 0):
            raise ValueError("topk selection needs positive topk_communities and max_selected")
        if self.assignment not in ASSIGNMENT_MODES:
            raise ValueError(f"assignment must be one of {ASSIGNMENT_MODES}")


@dataclass(frozen=True, slots=True)
class PartitionConfig:
    """Prefill partition scheduling (reference config.py:61-70).  ``devices``
    names GPUs for partition offload (only the model's own GPU is supported
    here); ``overlap`` (this build's switch) runs each layer's partition on a
    worker thread and its own stream so that it overlaps the prefill of later
    layers, as the reference's worker pool does; ``False`` runs it inline."""

    devices: tuple[str, ...] = ()
    workers_per_device: int = 2
    overlap: bool = True

    def __post_init__(self) -> None:
        if self.workers_per_device <= 0:
            raise ValueError("workers_per_device must be positive")


__all__ = ["CommunityKVConfig", "GraphAggregation", "PartitionConfig"]
