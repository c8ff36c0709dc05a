"""CommunityKV sparse decode for AMD Instinct MI355X (gfx950).

Public API mirrors the reference package ``community_kv`` (its ``__all__``,
community_kv/__init__.py:18-32): register the attention plugin with
``CommunityKVAttention(runtime).register()`` and generate with
``CommunityKVRuntime.generate``.  Kernels live in ``libckv_amd.so``
(``include/ckv_amd.h``), built by ``community_kv_amd._native.build()``.
"""

from community_kv_amd.attention.adapter import ATTENTION_IMPLEMENTATION, CommunityKVAttention, HuggingFaceAttention
from community_kv_amd.attention.cache import StaticCache, StaticCacheLayer
from community_kv_amd.attention.flash_attention import prefill_attention_topk
from community_kv_amd.config import CommunityKVConfig, GraphAggregation, PartitionConfig
from community_kv_amd.graph.partition import leiden_max_iterations, partition_graphs, partition_query_groups
from community_kv_amd.runtime import CommunityKVRuntime

__all__ = [
    "ATTENTION_IMPLEMENTATION",
    "CommunityKVAttention",
    "CommunityKVConfig",
    "CommunityKVRuntime",
    "GraphAggregation",
    "HuggingFaceAttention",
    "PartitionConfig",
    "StaticCache",
    "StaticCacheLayer",
    "leiden_max_iterations",
    "partition_graphs",
    "partition_query_groups",
    "prefill_attention_topk",
]
