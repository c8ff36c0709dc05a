"""Attention adapters, cache types, selection, and decode primitives."""

from community_kv_amd.attention.adapter import ATTENTION_IMPLEMENTATION, CommunityKVAttention, HuggingFaceAttention
from community_kv_amd.attention.cache import StaticCache, StaticCacheLayer
from community_kv_amd.attention.decode import DecodeLayerWorkspace, decode_layer
from community_kv_amd.attention.flash_attention import prefill_attention_topk
from community_kv_amd.attention.kernels.packed_segments import PackedSegments

__all__ = [
    "ATTENTION_IMPLEMENTATION",
    "CommunityKVAttention",
    "DecodeLayerWorkspace",
    "HuggingFaceAttention",
    "PackedSegments",
    "StaticCache",
    "StaticCacheLayer",
    "decode_layer",
    "prefill_attention_topk",
]
