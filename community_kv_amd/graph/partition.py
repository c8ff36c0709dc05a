"""Decode-state assembly from community labels (reference: community_kv/graph/partition.py).

These builders run once per request (not per token).  They turn per-token
community labels and the prefill keys into the tensors the decode kernels use:
FP8 centroids with decode headroom, the recency-descending member CSR, and the
modularity weights.  ``build_adjacency`` restates the reference's top-k edge
graph; ``partition_graphs`` runs the native batched Leiden on it
(``graph.leiden``) and ``build_partitioned_layer`` chains the two with the
state build.  Callers may also supply labels directly through
``build_layer_from_labels`` or a ``PartitionRuntime`` label provider.
"""

from __future__ import annotations

from typing import Any

import math
from dataclasses import dataclass, fields, replace

import torch

from community_kv_amd.config import GraphAggregation


def leiden_max_iterations(input_context_length: int) -> int:
    """Leiden sweep limit for a context length (partition.py:14-23)."""
    if (not isinstance(input_context_length, int) or isinstance(input_context_length, bool)
            or input_context_length <= 0):
        raise ValueError("input_context_length must be a positive integer")
    return max(1, math.floor(math.log10(input_context_length)))


@dataclass(slots=True)
class PartitionResult:
    community_ids: torch.Tensor
    community_counts: torch.Tensor
    modularity: float
    edge_src: torch.Tensor
    edge_dst: torch.Tensor
    edge_weight: torch.Tensor


@dataclass(slots=True)
class PartitionedLayer:
    """Compact per-layer tensors handed to the decode runtime (partition.py:36-68)."""

    layer_idx: int
    prefill_seq_len: int
    aggregation: GraphAggregation
    query_heads: int
    kv_heads: int
    retrieval_to_graph: torch.Tensor
    retrieval_to_kv: torch.Tensor
    member_offsets: torch.Tensor
    member_positions: torch.Tensor
    community_counts: torch.Tensor
    centroids: torch.Tensor
    community_sizes: torch.Tensor
    community_weight: torch.Tensor
    total_weight: torch.Tensor
    token_communities: torch.Tensor

    def to(self, device: torch.device | str, *, non_blocking: bool = False) -> "PartitionedLayer":
        target = torch.device(device)
        updates = {f.name: getattr(self, f.name).to(target, non_blocking=non_blocking)
                   for f in fields(self) if isinstance(getattr(self, f.name), torch.Tensor)}
        return replace(self, **updates)


def aggregation_mappings(aggregation: GraphAggregation, *, query_heads: int, kv_heads: int,
                         device: torch.device | str) -> tuple[torch.Tensor, torch.Tensor]:
    """Retrieval head -> (graph, KV head) (partition.py:71-94)."""
    aggregation = GraphAggregation(aggregation)
    count = aggregation.retrieval_head_count(query_heads=query_heads, kv_heads=kv_heads)
    heads = torch.arange(count, dtype=torch.int32, device=device)
    if aggregation is GraphAggregation.PER_QUERY_HEAD:
        return heads, heads // (query_heads // kv_heads)
    if aggregation is GraphAggregation.QUERY_GROUP:
        return heads, heads.clone()
    return torch.zeros_like(heads), heads


def build_adjacency(topk_indices: torch.Tensor, topk_scores: torch.Tensor, query_positions: torch.Tensor,
                    *, seq_len: int, lam: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Coalesced disjoint batched token graph from top-k edges (partition.py:168-249):
    direct edges weighted lam/2 * p, co-occurrence edges (1 - lam) * p_i * p_j.
    Device tensors run ``ckv_build_adjacency`` (one radix sort of the edge
    keys, equal pairs summed); the torch ops below serve host tensors."""
    if topk_indices.device.type == "cuda":
        return _native_adjacency(topk_indices, topk_scores, query_positions, seq_len=seq_len, lam=lam)
    graphs, _, kappa = topk_indices.shape
    device = topk_indices.device
    total = graphs * seq_len
    offset = torch.arange(graphs, device=device, dtype=torch.int64).unsqueeze(1) * seq_len
    src = (query_positions.long() + offset).unsqueeze(-1).expand_as(topk_indices)
    dst = topk_indices.long() + offset.unsqueeze(-1)
    ok = (topk_indices >= 0) & (topk_indices < seq_len)
    a_src, a_dst, a_w = [src[ok]], [dst[ok]], [topk_scores.float()[ok] * (lam / 2.0)]
    if lam < 1.0:
        row, col = torch.triu_indices(kappa, kappa, device=device)
        ci, cj = topk_indices[..., row], topk_indices[..., col]
        ok2 = (ci >= 0) & (ci < seq_len) & (cj >= 0) & (cj < seq_len)
        a_src.append((ci.long() + offset.unsqueeze(-1))[ok2])
        a_dst.append((cj.long() + offset.unsqueeze(-1))[ok2])
        a_w.append((topk_scores[..., row].float() * topk_scores[..., col].float())[ok2] * (1.0 - lam))
    s = torch.cat(a_src)
    d = torch.cat(a_dst)
    lo, hi = torch.minimum(s, d), torch.maximum(s, d)
    keys = lo * total + hi
    unique, inverse = keys.unique(return_inverse=True)
    weight = torch.zeros(unique.shape[0], dtype=torch.float32, device=device)
    weight.scatter_add_(0, inverse, torch.cat(a_w))
    return (unique // total).to(torch.int32), (unique % total).to(torch.int32), weight


def _native_adjacency(topk_indices: torch.Tensor, topk_scores: torch.Tensor, query_positions: torch.Tensor, *,
                      seq_len: int, lam: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    from community_kv_amd import _native as nat

    device = nat.require_device(topk_indices, topk_scores, query_positions)
    graphs, rows, kappa = topk_indices.shape
    idx = topk_indices.to(torch.int32).contiguous()
    sc = topk_scores.to(torch.float32).contiguous()
    pos = query_positions.to(torch.int64).expand(graphs, rows).contiguous()
    lib = nat.lib()
    cap = lib.ckv_adjacency_capacity(graphs, rows, kappa, float(lam))
    out_src = torch.empty(max(cap, 1), dtype=torch.int32, device=device)
    out_dst = torch.empty(max(cap, 1), dtype=torch.int32, device=device)
    out_w = torch.empty(max(cap, 1), dtype=torch.float32, device=device)
    count = torch.zeros(1, dtype=torch.int64, device=device)
    ws = torch.empty(max(1, (lib.ckv_adjacency_workspace_bytes(graphs, rows, kappa, float(lam)) + 7) // 8),
                     dtype=torch.int64, device=device)
    nat.check(lib.ckv_build_adjacency(nat.ptr(idx), nat.ptr(sc), nat.ptr(pos), graphs, rows, kappa, seq_len,
                                      float(lam), nat.ptr(out_src), nat.ptr(out_dst), nat.ptr(out_w), nat.ptr(count),
                                      nat.ptr(ws), nat.stream_handle(device)))
    n = int(count.item())
    return out_src[:n], out_dst[:n], out_w[:n]


def compute_centroids(community_ids: torch.Tensor, community_counts: torch.Tensor, keys: torch.Tensor, *,
                      retrieval_to_graph: torch.Tensor | None = None,
                      retrieval_to_kv: torch.Tensor | None = None, num_sink: int,
                      max_decode_tokens: int, fp8: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-retrieval-head centroid tables: mean of each community's non-sink
    keys, clamped to +-448 and stored as FP8 E4M3, with ``max_decode_tokens``
    rows of headroom (partition.py:382-454)."""
    graphs, seq_len = community_ids.shape
    if keys.ndim != 3 or keys.shape[1] != seq_len:
        raise ValueError("keys must have shape [KV heads, sequence, head dim]")
    if retrieval_to_graph is None or retrieval_to_kv is None:
        if keys.shape[0] != graphs:
            raise ValueError("aggregation mappings are required when graph and KV counts differ")
        retrieval_to_graph = torch.arange(graphs, dtype=torch.int32, device=community_ids.device)
        retrieval_to_kv = retrieval_to_graph
    heads = retrieval_to_graph.numel()
    active = int(community_counts.max().item())
    capacity = active + max_decode_tokens
    dim = keys.shape[-1]
    sums = torch.zeros((heads, capacity, dim), dtype=torch.float32, device=keys.device)
    sizes = torch.zeros((heads, capacity), dtype=torch.int32, device=keys.device)
    ids = community_ids[retrieval_to_graph.long(), num_sink:].long()
    sums.scatter_add_(1, ids.unsqueeze(-1).expand(-1, -1, dim), keys[retrieval_to_kv.long(), num_sink:].float())
    sizes.scatter_add_(1, ids, torch.ones_like(ids, dtype=torch.int32))
    sums[:, :active].div_(sizes[:, :active].float().clamp_min(1).unsqueeze(-1))
    limit = torch.finfo(torch.float8_e4m3fn).max
    sums.clamp_(min=-limit, max=limit)
    return (sums.to(torch.float8_e4m3fn) if fp8 else sums), sizes


def build_member_csr(community_ids: torch.Tensor, community_counts: torch.Tensor, *,
                     num_sink: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Recency-descending membership CSR over non-sink positions (partition.py:457-492)."""
    graphs, seq_len = community_ids.shape
    maxc = int(community_counts.max().item())
    ids = community_ids[:, num_sink:].long()
    positions = torch.arange(num_sink, seq_len, dtype=torch.int64,
                             device=community_ids.device).unsqueeze(0).expand(graphs, -1)
    order = (ids * seq_len + (seq_len - 1 - positions)).argsort(dim=1)
    member_positions = torch.gather(positions, 1, order).to(torch.int32)
    counts = torch.zeros((graphs, maxc), dtype=torch.int64, device=community_ids.device)
    counts.scatter_add_(1, ids, torch.ones_like(ids))
    offsets = torch.zeros((graphs, maxc + 1), dtype=torch.int32, device=community_ids.device)
    offsets[:, 1:] = counts.cumsum(dim=1).to(torch.int32)
    return offsets, member_positions


def init_modularity_state(result: PartitionResult, *, community_capacity: int,
                          seq_len: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Community degree weights and 2m from the coalesced edges (partition.py:495-535)."""
    graphs = result.community_ids.shape[0]
    device = result.community_ids.device
    weight = torch.zeros((graphs, community_capacity), dtype=torch.float32, device=device)
    total = torch.zeros((graphs,), dtype=torch.float32, device=device)
    if not result.edge_src.numel():
        return weight, total
    src = result.edge_src.long()
    dst = result.edge_dst.long()
    graph = src // seq_len
    sc = result.community_ids[graph, src % seq_len].long()
    dc = result.community_ids[graph, dst % seq_len].long()
    w = result.edge_weight.float()
    flat = weight.view(-1)
    flat.scatter_add_(0, graph * community_capacity + sc, w)
    flat.scatter_add_(0, graph * community_capacity + dc, w)
    total.scatter_add_(0, graph, 2.0 * w)
    return weight, total


def build_layer_from_labels(*, layer_idx: int, community_ids: torch.Tensor, keys: torch.Tensor,
                            num_sink: int, max_decode_tokens: int, query_heads: int,
                            aggregation: GraphAggregation = GraphAggregation.PER_QUERY_HEAD,
                            edges: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
                            fp8: bool = True, topk_edges: Any = None,
                            count_sink_labels: bool = False) -> PartitionedLayer:
    """Everything ``build_partitioned_layer`` (partition.py:538-618) produces
    after Leiden, from given dense labels ``community_ids [graphs, S]``.  The
    modularity weights come from ``edges`` (a coalesced edge list) or from
    ``topk_edges`` (a ``graph.kernels.state_build.TopkEdges``: the prefill
    top-k edges, device tensors only), or are zero.  The community count is
    1 + the largest non-sink label, or, with ``count_sink_labels``, 1 + the
    largest label of any position (the reference's count after Leiden, whose
    sink singletons may carry the largest ids)."""
    if max_decode_tokens <= 0:
        raise ValueError("max_decode_tokens must be positive")
    kv_heads, seq_len, _ = keys.shape
    aggregation = GraphAggregation(aggregation)
    to_graph, to_kv = aggregation_mappings(aggregation, query_heads=query_heads, kv_heads=kv_heads,
                                           device=keys.device)
    ids = community_ids.to(device=keys.device, dtype=torch.int32)
    if keys.device.type == "cuda":
        # HIP kernels (graph/kernels/state_build.py); the torch code below
        # serves CPU tensors only
        from community_kv_amd.graph.kernels.state_build import build_layer_state

        st = build_layer_state(ids, keys, retrieval_to_graph=to_graph, retrieval_to_kv=to_kv, num_sink=num_sink,
                               max_decode_tokens=max_decode_tokens, fp8=fp8, edges=edges, topk_edges=topk_edges,
                               count_sink_labels=count_sink_labels)
        return PartitionedLayer(layer_idx=layer_idx, prefill_seq_len=seq_len, aggregation=aggregation,
                                query_heads=query_heads, kv_heads=kv_heads, retrieval_to_graph=to_graph,
                                retrieval_to_kv=to_kv, member_offsets=st.member_offsets,
                                member_positions=st.member_positions, community_counts=st.community_counts,
                                centroids=st.centroids, community_sizes=st.community_sizes,
                                community_weight=st.community_weight, total_weight=st.total_weight,
                                token_communities=st.token_communities)
    if topk_edges is not None:
        raise ValueError("top-k edges are taken by the device state build only; pass a coalesced edge list")
    counts = (ids[:, 0 if count_sink_labels else num_sink:].amax(dim=1) + 1).to(torch.int32)
    centroids, sizes = compute_centroids(ids, counts, keys, retrieval_to_graph=to_graph, retrieval_to_kv=to_kv,
                                         num_sink=num_sink, max_decode_tokens=max_decode_tokens, fp8=fp8)
    offsets, positions = build_member_csr(ids, counts, num_sink=num_sink)
    empty_i = torch.zeros(0, dtype=torch.int32, device=keys.device)
    src, dst, w = edges if edges is not None else (empty_i, empty_i, torch.zeros(0, device=keys.device))
    result = PartitionResult(ids, counts, 0.0, src, dst, w)
    weight, total = init_modularity_state(result, community_capacity=centroids.shape[1], seq_len=seq_len)
    tokens = torch.full((ids.shape[0], seq_len + max_decode_tokens), -1, dtype=torch.int32, device=keys.device)
    tokens[:, :seq_len].copy_(ids)
    return PartitionedLayer(layer_idx=layer_idx, prefill_seq_len=seq_len, aggregation=aggregation,
                            query_heads=query_heads, kv_heads=kv_heads, retrieval_to_graph=to_graph,
                            retrieval_to_kv=to_kv, member_offsets=offsets, member_positions=positions,
                            community_counts=counts, centroids=centroids, community_sizes=sizes,
                            community_weight=weight, total_weight=total, token_communities=tokens)


def _reshape_by_aggregation(topk_indices: torch.Tensor, topk_scores: torch.Tensor, *,
                            aggregation: GraphAggregation, num_kv_heads: int,
                            num_sink: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Top-k rows grouped into graphs (partition.py:97-147): per query head,
    per KV-head group, or one graph; row r is position kappa - 1 + num_sink + r."""
    if topk_indices.ndim != 3 or topk_scores.shape != topk_indices.shape:
        raise ValueError("top-k tensors must have shape [query heads, rows, kappa]")
    query_heads, rows, kappa = topk_indices.shape
    if num_kv_heads <= 0 or query_heads % num_kv_heads:
        raise ValueError("query heads must divide evenly into KV-head groups")
    group = query_heads // num_kv_heads
    if not 1 <= group <= 16:
        raise ValueError("GQA group size must be in [1, 16]")
    base = torch.arange(kappa - 1 + num_sink, kappa - 1 + num_sink + rows, dtype=torch.int64,
                        device=topk_indices.device)
    aggregation = GraphAggregation(aggregation)
    if aggregation is GraphAggregation.PER_QUERY_HEAD:
        return topk_indices, topk_scores, base.unsqueeze(0).expand(query_heads, -1)
    if aggregation is GraphAggregation.QUERY_GROUP:
        shape = (num_kv_heads, group * rows, kappa)
        return (topk_indices.reshape(shape), topk_scores.reshape(shape),
                base.repeat(group).unsqueeze(0).expand(num_kv_heads, -1))
    return (topk_indices.reshape(1, query_heads * rows, kappa), topk_scores.reshape(1, query_heads * rows, kappa),
            base.repeat(query_heads).unsqueeze(0))


def _scatter_membership(vertex: torch.Tensor, labels: torch.Tensor, *, graph_count: int,
                        seq_len: int) -> torch.Tensor:
    """partition.py:252-266: Leiden labels into a [graphs, S] table, -1 elsewhere."""
    membership = torch.full((graph_count * seq_len,), -1, dtype=torch.int32, device=vertex.device)
    membership[vertex] = labels
    return membership.view(graph_count, seq_len)


def _fill_isolated_vertices(membership: torch.Tensor) -> torch.Tensor:
    """partition.py:269-273: vertices without edges become singletons numbered
    after the graph's largest label, in position order."""
    missing = membership == -1
    next_ids = membership.amax(dim=1) + 1
    offsets = missing.to(torch.int32).cumsum(dim=1) - 1
    return torch.where(missing, next_ids.unsqueeze(1) + offsets, membership)


def _dense_remap(membership: torch.Tensor) -> torch.Tensor:
    """partition.py:276-286: per graph, each label becomes its rank among the
    graph's distinct labels."""
    sorted_values, order = membership.sort(dim=-1)
    transitions = torch.ones_like(sorted_values, dtype=torch.int32)
    if sorted_values.shape[-1] > 1:
        transitions[:, 1:] = (sorted_values[:, 1:] != sorted_values[:, :-1]).to(torch.int32)
    dense = torch.empty_like(membership, dtype=torch.int32)
    dense.scatter_(1, order, (transitions.cumsum(dim=-1) - 1).to(torch.int32))
    return dense


def partition_graphs(topk_indices: torch.Tensor, topk_scores: torch.Tensor, *, aggregation: GraphAggregation,
                     num_kv_heads: int, prefill_seq_len: int, num_sink: int, lam: float, leiden_resolution: float,
                     leiden_seed: int) -> PartitionResult:
    """Top-k edges -> coalesced graph -> native batched Leiden -> dense
    per-graph community ids (partition.py:289-353).  Device tensors only."""
    from community_kv_amd.graph.leiden import run_leiden

    grouped_idx, grouped_scores, positions = _reshape_by_aggregation(
        topk_indices, topk_scores, aggregation=aggregation, num_kv_heads=num_kv_heads, num_sink=num_sink)
    graph_count = grouped_idx.shape[0]
    src, dst, weight = build_adjacency(grouped_idx, grouped_scores, positions, seq_len=prefill_seq_len, lam=lam)
    if src.numel():
        vertex, labels, modularity = run_leiden(src, dst, weight, G=graph_count, seq_len=prefill_seq_len,
                                                resolution=leiden_resolution,
                                                max_inner_iter=leiden_max_iterations(prefill_seq_len),
                                                seed=leiden_seed)
        membership = _scatter_membership(vertex, labels, graph_count=graph_count, seq_len=prefill_seq_len)
    else:
        modularity = 0.0
        membership = torch.full((graph_count, prefill_seq_len), -1, dtype=torch.int32, device=topk_indices.device)
    community_ids = _dense_remap(_fill_isolated_vertices(membership))
    community_counts = (community_ids.amax(dim=1) + 1).to(torch.int32)
    return PartitionResult(community_ids=community_ids, community_counts=community_counts, modularity=modularity,
                           edge_src=src, edge_dst=dst, edge_weight=weight)


def partition_query_groups(topk_indices: torch.Tensor, topk_scores: torch.Tensor, *, num_kv_heads: int,
                           prefill_seq_len: int, num_sink: int, lam: float, leiden_resolution: float,
                           leiden_seed: int) -> PartitionResult:
    """Query-group wrapper of :func:`partition_graphs` (partition.py:356-379)."""
    return partition_graphs(topk_indices, topk_scores, aggregation=GraphAggregation.QUERY_GROUP,
                            num_kv_heads=num_kv_heads, prefill_seq_len=prefill_seq_len, num_sink=num_sink, lam=lam,
                            leiden_resolution=leiden_resolution, leiden_seed=leiden_seed)


def build_partitioned_layer(*, layer_idx: int, topk_indices: torch.Tensor, topk_scores: torch.Tensor,
                            keys: torch.Tensor, num_sink: int, lam: float, leiden_resolution: float,
                            leiden_seed: int, max_decode_tokens: int,
                            aggregation: GraphAggregation = GraphAggregation.PER_QUERY_HEAD) -> PartitionedLayer:
    """Full prefill partition of one layer and its decode state
    (partition.py:538-618): Leiden on the top-k graph, then the state build
    with the community count over all positions, sinks included, as the
    reference counts them."""
    if max_decode_tokens <= 0:
        raise ValueError("max_decode_tokens must be positive")
    kv_heads, seq_len, _ = keys.shape
    aggregation = GraphAggregation(aggregation)
    result = partition_graphs(topk_indices, topk_scores, aggregation=aggregation, num_kv_heads=kv_heads,
                              prefill_seq_len=seq_len, num_sink=num_sink, lam=lam,
                              leiden_resolution=leiden_resolution, leiden_seed=leiden_seed)
    edges = (result.edge_src, result.edge_dst, result.edge_weight) if result.edge_src.numel() else None
    return build_layer_from_labels(layer_idx=layer_idx, community_ids=result.community_ids, keys=keys,
                                   num_sink=num_sink, max_decode_tokens=max_decode_tokens,
                                   query_heads=topk_indices.shape[0], aggregation=aggregation, edges=edges,
                                   count_sink_labels=True)


__all__ = [
    "PartitionResult", "PartitionedLayer", "aggregation_mappings", "build_adjacency", "build_layer_from_labels",
    "build_partitioned_layer",
    "build_member_csr", "compute_centroids", "init_modularity_state", "leiden_max_iterations",
    "partition_graphs", "partition_query_groups",
]
