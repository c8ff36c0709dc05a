"""Seeded graphs for the Leiden tests (upper-triangular COO over G disjoint
graphs, vertex ids g * seq_len + i)."""

from __future__ import annotations

import numpy as np


def planted(seed: int, graphs: int, seq_len: int, communities: int, *, edges_per_vertex: float = 4.0,
            p_in: float = 0.85, dyadic: bool = True, self_loops: int = 0, isolated: int = 0,
            duplicates: int = 0):
    """Planted-partition graphs.  Dyadic weights (k/16, k in 1..63) make every
    float sum exact.  The last ``isolated`` vertices of each graph get no edges."""
    rng = np.random.default_rng(seed)
    src, dst = [], []
    live = seq_len - isolated
    for g in range(graphs):
        comm = rng.integers(0, communities, live)
        n = int(edges_per_vertex * live)
        a = rng.integers(0, live, n)
        same = rng.random(n) < p_in
        b = np.empty(n, np.int64)
        for i in range(n):
            if same[i]:
                members = np.nonzero(comm == comm[a[i]])[0]
                b[i] = members[rng.integers(0, members.size)]
            else:
                b[i] = rng.integers(0, live)
        keep = a != b
        a, b = a[keep], b[keep]
        lo, hi = np.minimum(a, b), np.maximum(a, b)
        key = np.unique(lo * seq_len + hi)
        lo, hi = key // seq_len, key % seq_len
        if self_loops:
            s = rng.choice(live, self_loops, replace=False)
            lo, hi = np.concatenate([lo, s]), np.concatenate([hi, s])
        if duplicates:
            d = rng.integers(0, lo.size, duplicates)
            lo, hi = np.concatenate([lo, lo[d]]), np.concatenate([hi, hi[d]])
        src.append(lo + g * seq_len)
        dst.append(hi + g * seq_len)
    src = np.concatenate(src).astype(np.int32)
    dst = np.concatenate(dst).astype(np.int32)
    if dyadic:
        w = (rng.integers(1, 64, src.size) / 16.0).astype(np.float32)
    else:
        w = rng.random(src.size).astype(np.float32) + np.float32(0.01)
    return src, dst, w


def ring_of_cliques(graphs: int, cliques: int, size: int, seq_len: int | None = None):
    """Cliques of ``size`` joined in a ring by single edges; vertices past
    cliques * size are isolated."""
    seq_len = seq_len or cliques * size
    src, dst = [], []
    for g in range(graphs):
        for k in range(cliques):
            base = g * seq_len + k * size
            for i in range(size):
                for j in range(i + 1, size):
                    src.append(base + i)
                    dst.append(base + j)
            src.append(base + size - 1)
            dst.append(g * seq_len + ((k + 1) % cliques) * size)
    src = np.asarray(src, np.int64)
    dst = np.asarray(dst, np.int64)
    lo, hi = np.minimum(src, dst), np.maximum(src, dst)
    return lo.astype(np.int32), hi.astype(np.int32), np.ones(lo.size, np.float32), seq_len


def hub(seed: int, leaves: int, groups: int):
    """One graph: vertex 0 joined to every leaf, leaves in ``groups`` chains
    (a hub with more distinct neighbour communities than a 64-lane chunk and,
    at the first sweep, than the 1024-entry table)."""
    rng = np.random.default_rng(seed)
    S = leaves + 1
    src = [np.zeros(leaves, np.int64)]
    dst = [np.arange(1, S)]
    order = rng.permutation(np.arange(1, S))
    for chunk in np.array_split(order, groups):
        src.append(chunk[:-1])
        dst.append(chunk[1:])
    s, d = np.concatenate(src), np.concatenate(dst)
    lo, hi = np.minimum(s, d), np.maximum(s, d)
    w = (rng.integers(1, 64, lo.size) / 16.0).astype(np.float32)
    return lo.astype(np.int32), hi.astype(np.int32), w, S
