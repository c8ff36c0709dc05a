"""Batched Leiden on the GPU (reference: community_kv/graph/leiden)."""

from community_kv_amd.graph.leiden.algorithm import run_leiden

__all__ = ["run_leiden"]
