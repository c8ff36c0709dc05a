"""GPU state assembly from dense community labels (HIP kernels of
``ckv_label_counts`` / ``ckv_build_layer_state``).

Produces what the reference's ``build_partitioned_layer`` builds after Leiden
(graph/partition.py:538-618): ``compute_centroids`` (382-454),
``build_member_csr`` (457-492), ``init_modularity_state`` (495-535) and the
token-community table.  The CSR and the sizes are exact; the centroid sums add
keys in ascending position order in blocks of 64 (reproducible bit for bit);
the modularity weights use float atomics like the reference's
``scatter_add_``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from community_kv_amd import _native as nat


@dataclass
class TopkEdges:
    """Prefill top-k edges as the partitioner receives them: ``indices`` /
    ``scores`` ``[heads, rows, kappa]`` with heads grouped by graph (``group``
    query heads per graph); row r is position ``row0 + r``.  The state build
    derives the modularity weights of the reference's ``build_adjacency``
    graph (partition.py:168-249, weight ``lam``) from them directly."""
    indices: torch.Tensor
    scores: torch.Tensor
    row0: int
    group: int
    lam: float


@dataclass
class LayerStateTensors:
    community_counts: torch.Tensor   # int32 [graphs]
    member_offsets: torch.Tensor     # int32 [graphs, maxc + 1]
    member_positions: torch.Tensor   # int32 [graphs, S - num_sink]
    centroids: torch.Tensor          # float8_e4m3fn or float32 [R, capacity, 128]
    community_sizes: torch.Tensor    # int32 [R, capacity]
    community_weight: torch.Tensor   # float32 [graphs, capacity]
    total_weight: torch.Tensor       # float32 [graphs]
    token_communities: torch.Tensor  # int32 [graphs, token_capacity]


def label_counts(community_ids: torch.Tensor, *, num_sink: int) -> torch.Tensor:
    """1 + the largest non-sink label per graph (``ckv_label_counts``)."""
    nat.require_device(community_ids)
    if community_ids.dtype != torch.int32 or community_ids.ndim != 2 or not community_ids.is_contiguous():
        raise TypeError("community_ids must be a contiguous int32 [graphs, seq_len] tensor")
    graphs, seq_len = community_ids.shape
    counts = torch.empty(graphs, dtype=torch.int32, device=community_ids.device)
    nat.check(nat.lib().ckv_label_counts(nat.ptr(community_ids), graphs, seq_len, num_sink, nat.ptr(counts),
                                         nat.stream_handle(community_ids.device)))
    return counts


class StateBuild:
    """One layer's state build, set up once: reads the community counts back,
    allocates the outputs and the workspace, and packs the launch arguments;
    ``run()`` queues ``ckv_build_layer_state`` on the current stream (it may be
    replayed, e.g. for timing)."""

    def __init__(self, community_ids: torch.Tensor, keys: torch.Tensor, *, retrieval_to_graph: torch.Tensor,
                 retrieval_to_kv: torch.Tensor, num_sink: int, max_decode_tokens: int, fp8: bool = True,
                 edges: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
                 token_capacity: int | None = None, topk_edges: "TopkEdges | None" = None,
                 count_sink_labels: bool = False):
        device = nat.require_device(community_ids, keys, retrieval_to_graph, retrieval_to_kv)
        if edges is not None and topk_edges is not None:
            raise ValueError("give either an edge list or top-k edges")
        if keys.ndim != 3 or keys.shape[-1] != nat.HEAD_DIM or keys.stride(-1) != 1:
            raise ValueError("keys must be [KV heads, sequence, 128] with unit dim stride")
        graphs, seq_len = community_ids.shape
        if keys.shape[1] < seq_len:
            raise ValueError("keys must cover the labelled sequence")
        if not 0 <= num_sink < seq_len:
            raise ValueError("num_sink must be below the sequence length")
        if retrieval_to_graph.dtype != torch.int32 or retrieval_to_kv.dtype != torch.int32:
            raise TypeError("aggregation mappings must be int32")
        self.device = device
        self.ids = community_ids.to(torch.int32).contiguous()
        counts = label_counts(self.ids, num_sink=0 if count_sink_labels else num_sink)
        host_counts = counts.cpu()
        if int(host_counts.min()) < 0:
            raise ValueError("community labels of non-sink positions must be nonnegative")
        maxc = int(host_counts.max())
        if maxc <= 0:
            raise ValueError("no labelled non-sink positions")
        if maxc > nat.MAX_COMMUNITIES:
            raise ValueError(f"more than {nat.MAX_COMMUNITIES} communities per graph are not supported")
        capacity = maxc + max_decode_tokens
        token_capacity = seq_len + max_decode_tokens if token_capacity is None else token_capacity
        heads = retrieval_to_graph.numel()
        lib = nat.lib()
        ws_bytes = lib.ckv_state_workspace_bytes(graphs, heads, seq_len, num_sink, maxc)
        i32 = dict(dtype=torch.int32, device=device)
        self.out = LayerStateTensors(
            community_counts=counts,
            member_offsets=torch.empty((graphs, maxc + 1), **i32),
            member_positions=torch.empty((graphs, seq_len - num_sink), **i32),
            centroids=torch.empty((heads, capacity, nat.HEAD_DIM),
                                  dtype=torch.float8_e4m3fn if fp8 else torch.float32, device=device),
            community_sizes=torch.empty((heads, capacity), **i32),
            community_weight=torch.empty((graphs, capacity), dtype=torch.float32, device=device),
            total_weight=torch.empty((graphs,), dtype=torch.float32, device=device),
            token_communities=torch.empty((graphs, token_capacity), **i32),
        )
        self.workspace = torch.empty(max(ws_bytes // 4, 1), **i32)
        self.keys = keys
        self.edges = None
        n_edges = 0
        if edges is not None and edges[0].numel():
            self.edges = (edges[0].to(device=device, dtype=torch.int32).contiguous(),
                          edges[1].to(device=device, dtype=torch.int32).contiguous(),
                          edges[2].to(device=device, dtype=torch.float32).contiguous())
            n_edges = self.edges[0].numel()
        src, dst, w = self.edges if self.edges is not None else (None, None, None)
        self.topk = None
        tk = dict(topk_indices=None, topk_scores=None, topk_heads=0, topk_rows=0, topk_kappa=0, topk_group=1,
                  topk_row0=0, lam=0.0)
        if topk_edges is not None:
            ti = topk_edges.indices.to(device=device, dtype=torch.int32).contiguous()
            ts = topk_edges.scores.to(device=device, dtype=torch.float32).contiguous()
            if ti.ndim != 3 or ts.shape != ti.shape or ti.shape[-1] > 16:
                raise ValueError("top-k edges must be [heads, rows, kappa <= 16] indices with matching scores")
            if ti.shape[0] % graphs or ti.shape[0] // graphs != topk_edges.group:
                raise ValueError("top-k heads must be graphs x group, grouped by graph")
            self.topk = (ti, ts)
            tk = dict(topk_indices=nat.ptr(ti), topk_scores=nat.ptr(ts), topk_heads=ti.shape[0],
                      topk_rows=ti.shape[1], topk_kappa=ti.shape[2], topk_group=topk_edges.group,
                      topk_row0=topk_edges.row0, lam=float(topk_edges.lam))
        self.maps = (retrieval_to_graph.contiguous(), retrieval_to_kv.contiguous())
        o = self.out
        self.args = nat.StateBuildArgs(
            labels=nat.ptr(self.ids), keys=nat.ptr(keys), head_stride=keys.stride(0),
            token_stride=keys.stride(1), retrieval_to_graph=nat.ptr(self.maps[0]),
            retrieval_to_kv=nat.ptr(self.maps[1]), edge_src=nat.ptr(src), edge_dst=nat.ptr(dst),
            edge_weight=nat.ptr(w), edges=n_edges, graphs=graphs, seq_len=seq_len, num_sink=num_sink,
            retrieval_heads=heads, kv_heads=keys.shape[0], key_dtype=nat.dtype_code(keys.dtype),
            centroid_dtype=nat.CKV_E4M3 if fp8 else nat.CKV_F32, max_communities=maxc,
            community_capacity=capacity, token_capacity=token_capacity,
            member_offsets=nat.ptr(o.member_offsets), member_positions=nat.ptr(o.member_positions),
            centroids=nat.ptr(o.centroids), community_sizes=nat.ptr(o.community_sizes),
            community_weight=nat.ptr(o.community_weight), total_weight=nat.ptr(o.total_weight),
            token_communities=nat.ptr(o.token_communities), workspace=nat.ptr(self.workspace), **tk)

    def run(self) -> LayerStateTensors:
        nat.check(nat.lib().ckv_build_layer_state(self.args, nat.stream_handle(self.device)))
        return self.out


def build_layer_state(community_ids: torch.Tensor, keys: torch.Tensor, *, retrieval_to_graph: torch.Tensor,
                      retrieval_to_kv: torch.Tensor, num_sink: int, max_decode_tokens: int, fp8: bool = True,
                      edges: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
                      token_capacity: int | None = None, topk_edges: "TopkEdges | None" = None,
                      count_sink_labels: bool = False) -> LayerStateTensors:
    """Every prefill state tensor of one layer from labels ``[graphs, S]`` and
    keys ``[Hkv, S, 128]`` (bf16 or f32, token stride may exceed 128).  Reads
    the community counts back once to size the outputs, as the reference
    does with ``.item()``.  ``count_sink_labels`` counts communities over all
    positions (sinks included) instead of the non-sink ones.  (The workspace and edge copies return to the
    caching allocator on this stream, so later work on it cannot overwrite
    them before the launches run.)"""
    return StateBuild(community_ids, keys, retrieval_to_graph=retrieval_to_graph, retrieval_to_kv=retrieval_to_kv,
                      num_sink=num_sink, max_decode_tokens=max_decode_tokens, fp8=fp8, edges=edges,
                      token_capacity=token_capacity, topk_edges=topk_edges,
                      count_sink_labels=count_sink_labels).run()


__all__ = ["LayerStateTensors", "StateBuild", "TopkEdges", "build_layer_state", "label_counts"]
