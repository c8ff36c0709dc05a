"""Batched multi-level Leiden over the HIP kernels of ``ckv_leiden.hip``
(reference: community_kv/graph/leiden/algorithm.py:1-202).

Each level runs one ``ckv_batched_leiden`` (local moving + refinement, no host
round trips inside), densifies the labels per graph (``ckv_densify_count`` /
``ckv_densify_apply``) and contracts the edge list (``ckv_aggregate_coo``);
the chain of relabellings is composed back to the original vertices.  The
level loop reads two small device values per level (the densified width and
the aggregated edge count), as the reference does.
"""

from __future__ import annotations

import functools
import os

import torch

from community_kv_amd import _native as nat


class _Module:
    """The native entry points with the reference extension's Python
    signatures (graph/leiden/_csrc/bindings.cpp:40-181)."""

    @staticmethod
    def batched_leiden(edge_src: torch.Tensor, edge_dst: torch.Tensor, edge_weight: torch.Tensor, G: int,
                       seq_len: int, max_level: int = 6, resolution: float = 1.0, theta: float = 0.01,
                       max_inner_iter: int = 8, seed: int = 0, use_boltzmann: bool = False):
        device = nat.require_device(edge_src, edge_dst, edge_weight)
        _check_edges(edge_src, edge_dst, edge_weight)
        if G <= 0 or seq_len <= 0:
            raise RuntimeError("G and seq_len must be positive")
        lib = nat.lib()
        E = edge_src.numel()
        labels = torch.empty(G * seq_len, dtype=torch.int32, device=device)
        modularity = torch.empty(G, dtype=torch.float64, device=device)
        ws = torch.empty(max(1, (lib.ckv_leiden_workspace_bytes(E, G, seq_len) + 7) // 8), dtype=torch.int64,
                         device=device)
        nat.check(lib.ckv_batched_leiden(nat.ptr(edge_src), nat.ptr(edge_dst), nat.ptr(edge_weight), E, G, seq_len,
                                         float(resolution), float(theta), int(max_inner_iter), int(seed),
                                         1 if use_boltzmann else 0, nat.ptr(labels), nat.ptr(modularity),
                                         nat.ptr(ws), nat.stream_handle(device)))
        return labels, modularity

    @staticmethod
    def aggregate_coo(edge_src: torch.Tensor, edge_dst: torch.Tensor, edge_weight: torch.Tensor,
                      labels: torch.Tensor, V_super_total: int):
        device = nat.require_device(edge_src, edge_dst, edge_weight, labels)
        _check_edges(edge_src, edge_dst, edge_weight)
        if labels.dtype != torch.int32 or not labels.is_contiguous():
            raise RuntimeError("labels must be contiguous int32")
        if V_super_total <= 0:
            raise RuntimeError("V_super_total must be positive")
        lib = nat.lib()
        E = edge_src.numel()
        out_src = torch.empty(E, dtype=torch.int32, device=device)
        out_dst = torch.empty(E, dtype=torch.int32, device=device)
        out_w = torch.empty(E, dtype=torch.float32, device=device)
        count = torch.zeros(1, dtype=torch.int64, device=device)
        ws = torch.empty(max(1, (lib.ckv_aggregate_coo_workspace_bytes(E) + 7) // 8), dtype=torch.int64,
                         device=device)
        nat.check(lib.ckv_aggregate_coo(nat.ptr(edge_src), nat.ptr(edge_dst), nat.ptr(edge_weight), E,
                                        nat.ptr(labels), int(V_super_total), nat.ptr(out_src), nat.ptr(out_dst),
                                        nat.ptr(out_w), nat.ptr(count), nat.ptr(ws), nat.stream_handle(device)))
        n = int(count.item())
        return out_src[:n].contiguous(), out_dst[:n].contiguous(), out_w[:n].contiguous()


def _check_edges(src: torch.Tensor, dst: torch.Tensor, w: torch.Tensor) -> None:
    if src.dtype != torch.int32 or dst.dtype != torch.int32:
        raise RuntimeError("edge_src and edge_dst must be int32")
    if w.dtype != torch.float32:
        raise RuntimeError("edge_weight must be float32")
    if not (src.is_contiguous() and dst.is_contiguous() and w.is_contiguous()):
        raise RuntimeError("edge tensors must be contiguous")
    if src.numel() != dst.numel() or src.numel() != w.numel():
        raise RuntimeError("edge_src, edge_dst and edge_weight must have equal length")


@functools.cache
def _load_module() -> _Module:
    """The native library (loaded once; raises when it is not built)."""
    nat.lib()
    return _Module()


def _densify_per_graph(labels: torch.Tensor, G: int, seq_len: int) -> tuple[torch.Tensor, int]:
    """Per-graph dense relabel (algorithm.py:30-48): each label becomes its
    rank among the distinct labels of its graph, offset by g * width, width =
    the largest distinct count.  Labels are vertex ids inside their own graph
    (as Leiden produces them); negative labels stand for the vertex itself."""
    device = nat.require_device(labels)
    labels = labels.to(torch.int32).contiguous()
    if labels.numel() != G * seq_len:
        raise ValueError("labels must hold G * seq_len entries")
    lib = nat.lib()
    ws = torch.empty(max(1, (lib.ckv_densify_workspace_bytes(G, seq_len) + 7) // 8), dtype=torch.int64,
                     device=device)
    counts = torch.empty(G, dtype=torch.int32, device=device)
    stream = nat.stream_handle(device)
    nat.check(lib.ckv_densify_count(nat.ptr(labels), G, seq_len, nat.ptr(counts), nat.ptr(ws), stream))
    width = int(counts.max().item())
    dense = torch.empty(G * seq_len, dtype=torch.int32, device=device)
    nat.check(lib.ckv_densify_apply(nat.ptr(labels), G, seq_len, width, nat.ptr(dense), nat.ptr(ws), stream))
    return dense, width


def run_leiden(edge_src: torch.Tensor, edge_dst: torch.Tensor, edge_weight: torch.Tensor, *, G: int, seq_len: int,
               max_level: int = 6, resolution: float = 1.0, theta: float = 0.01, max_inner_iter: int = 16,
               seed: int = 0, use_boltzmann: bool = False) -> tuple[torch.Tensor, torch.Tensor, float]:
    """Multi-level Leiden over G vertex-disjoint graphs (algorithm.py:51-161).

    Returns (vertices that have edges, their final partition ids (dense per
    graph, offset by g * width of the last level), modularity of the disjoint
    union).  ``COMMUNITY_KV_LEIDEN_THETA``, ``COMMUNITY_KV_LEIDEN_MAX_INNER_ITER``
    and ``COMMUNITY_KV_LEIDEN_BOLTZMANN`` override the arguments, as in the
    reference."""
    module = _load_module()
    edge_src = edge_src.contiguous()
    edge_dst = edge_dst.contiguous()
    edge_weight = edge_weight.contiguous()
    V_orig = G * seq_len
    device = edge_src.device
    if edge_src.numel():
        # every edge inside one graph: the per-graph relabelling depends on it
        lo = torch.minimum(edge_src, edge_dst)
        bad = (lo < 0) | (torch.maximum(edge_src, edge_dst) >= V_orig) | (edge_src // seq_len != edge_dst // seq_len)
        if bool(bad.any()):
            raise ValueError("edges must join two vertices of the same graph, ids in [0, G * seq_len)")

    theta_env = os.environ.get("COMMUNITY_KV_LEIDEN_THETA")
    if theta_env is not None:
        theta = float(theta_env)
    iter_env = os.environ.get("COMMUNITY_KV_LEIDEN_MAX_INNER_ITER")
    if iter_env is not None:
        max_inner_iter = int(iter_env)
    boltzmann_env = os.environ.get("COMMUNITY_KV_LEIDEN_BOLTZMANN")
    if boltzmann_env is not None:
        use_boltzmann = boltzmann_env not in ("", "0", "false", "False")

    level_modularity = []
    labels0, mod0 = module.batched_leiden(edge_src, edge_dst, edge_weight, G, seq_len, max_level, float(resolution),
                                       float(theta), max_inner_iter, seed, use_boltzmann)
    level_modularity.append(mod0)
    is_isolated = labels0 == -1
    arange_v = torch.arange(V_orig, dtype=torch.int32, device=device)
    cur_labels = torch.where(is_isolated, arange_v, labels0)
    dense0, cur_seq_len = _densify_per_graph(cur_labels, G, seq_len)
    chain = dense0
    cur_src, cur_dst, cur_w = edge_src, edge_dst, edge_weight
    prev_seq_len = seq_len
    dense_for_agg = dense0
    for level in range(1, max_level):
        if cur_seq_len >= prev_seq_len:
            break
        cur_src, cur_dst, cur_w = module.aggregate_coo(cur_src, cur_dst, cur_w, dense_for_agg, G * cur_seq_len)
        if cur_src.numel() == 0:
            break
        labels_k, mod_k = module.batched_leiden(cur_src, cur_dst, cur_w, G, cur_seq_len, max_level,
                                                float(resolution), float(theta), max_inner_iter, seed + level,
                                                use_boltzmann)
        level_modularity.append(mod_k)
        arange_super = torch.arange(G * cur_seq_len, dtype=torch.int32, device=device)
        labels_k = torch.where(labels_k == -1, arange_super, labels_k)
        dense_k, next_seq_len = _densify_per_graph(labels_k, G, cur_seq_len)
        chain = dense_k[chain.long()]
        prev_seq_len = cur_seq_len
        cur_seq_len = next_seq_len
        dense_for_agg = dense_k

    # the native sweeps mark every graph's modularity NaN when a neighbour
    # table overflowed (a broken table bound): fail instead of returning labels
    if bool(torch.isnan(torch.cat(level_modularity)).any()):
        raise RuntimeError("Leiden: a neighbour-community table overflowed; the labels are not valid")
    modularity = _compute_disjoint_modularity(edge_src, edge_dst, edge_weight, chain, float(resolution))
    keep = ~is_isolated
    vertex = torch.nonzero(keep, as_tuple=False).squeeze(-1).long()
    return vertex, chain[keep].to(torch.int32), modularity


def _compute_disjoint_modularity(edge_src: torch.Tensor, edge_dst: torch.Tensor, edge_weight: torch.Tensor,
                                 labels: torch.Tensor, resolution: float) -> float:
    """Newman modularity of the disjoint union of the G graphs
    (algorithm.py:166-199): ``ckv_partition_modularity`` on device tensors
    (f64 sums), the same formula in float64 torch ops on host tensors."""
    if edge_src.numel() == 0:
        return 0.0
    if labels.device.type == "cuda":
        device = nat.require_device(edge_src, edge_dst, edge_weight, labels)
        lib = nat.lib()
        lab = labels.to(torch.int32).contiguous()
        V = lab.numel()
        ws = torch.empty(max(1, (lib.ckv_partition_modularity_workspace_bytes(V) + 7) // 8), dtype=torch.int64,
                         device=device)
        out = torch.empty(1, dtype=torch.float64, device=device)
        nat.check(lib.ckv_partition_modularity(nat.ptr(edge_src.contiguous()), nat.ptr(edge_dst.contiguous()),
                                               nat.ptr(edge_weight.contiguous()), edge_src.numel(), nat.ptr(lab), V,
                                               float(resolution), nat.ptr(out), nat.ptr(ws),
                                               nat.stream_handle(device)))
        return float(out.item())
    V = labels.numel()
    src = edge_src.long()
    dst = edge_dst.long()
    w64 = edge_weight.to(torch.float64)
    k = torch.zeros(V, dtype=torch.float64)
    k.scatter_add_(0, src, w64)
    k.scatter_add_(0, dst, w64)
    two_m = float(k.sum())
    if two_m <= 0.0:
        return 0.0
    lab = labels.long()
    in_total = 2.0 * float(w64[lab[src] == lab[dst]].sum())
    _, inverse = torch.unique(lab, return_inverse=True)
    sigma = torch.zeros(int(inverse.max()) + 1, dtype=torch.float64)
    sigma.scatter_add_(0, inverse, k)
    return in_total / two_m - resolution * float((sigma * sigma).sum()) / (two_m * two_m)


__all__ = ["run_leiden"]
