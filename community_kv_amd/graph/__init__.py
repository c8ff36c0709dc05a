"""Graph state layouts, decode-state assembly from labels, partition hand-off."""

from community_kv_amd.config import GraphAggregation
from community_kv_amd.graph.partition import (
    PartitionedLayer,
    PartitionResult,
    build_adjacency,
    build_layer_from_labels,
    build_member_csr,
    build_partitioned_layer,
    compute_centroids,
    init_modularity_state,
    leiden_max_iterations,
    partition_graphs,
    partition_query_groups,
)
from community_kv_amd.graph.runtime import PartitionRuntime
from community_kv_amd.graph.state import DecodeDeltaChunks, MutableGraphState, PrefillCSR

__all__ = [
    "DecodeDeltaChunks",
    "GraphAggregation",
    "MutableGraphState",
    "PartitionResult",
    "PartitionRuntime",
    "PartitionedLayer",
    "PrefillCSR",
    "build_adjacency",
    "build_layer_from_labels",
    "build_member_csr",
    "build_partitioned_layer",
    "compute_centroids",
    "init_modularity_state",
    "leiden_max_iterations",
    "partition_graphs",
    "partition_query_groups",
]
