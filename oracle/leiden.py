"""CPU restatement of the reference's batched Leiden (parity oracle).

TEST INFRASTRUCTURE ONLY: ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg
are the only callers; the product path (``community_kv_amd.graph.leiden``)
runs the HIP kernels of ``ckv_leiden.hip`` and never imports this module.

Restated from community_kv/graph/leiden/ (paths relative to the reference
repository root):

* ``build_csr`` -- csr.cu:20-271 (mirror non-self edges, self-loops once
  with doubled weight; k_v per vertex, 2m per graph).  Rows are ordered by
  neighbour id (the reference's radix sort leaves the order inside a row to
  its atomic counter; only the order of the first 1024 distinct neighbour
  communities can matter, see below).
* ``local_moving_sweep`` -- local_moving.cu:69-210: synchronous best-gain move
  on a snapshot, the up/down direction gate, the per-vertex jitter of
  rng.cuh:25-31, strict ``> 0`` gain.
* ``refine_propose`` / ``refine_commit`` -- refinement.cu:71-300: moves inside
  the local-moving community, the well-connectedness gate, greedy or Gumbel-max
  Boltzmann target, and the independent-set commit on (rank, id).
* ``batched_leiden`` -- leiden.cu:43-205 (sweep loop, up/down flip after a
  stalled sweep, two stalls end local moving; refinement from singletons).
* ``aggregate_coo`` -- aggregate.cu:24-184; ``densify_per_graph``,
  ``run_leiden`` and ``disjoint_modularity`` -- algorithm.py:30-202.

Tie rule between candidates of equal float score.  The reference scans a
1024-slot hash table with 128 threads (thread t takes slots t, t+128, ...,
keeping the first strict maximum) and reduces with 32-lane shuffle-down trees
that keep their own value on ties; a community's home slot is
``pcg_hash(c) & 1023``.  ``slot_key`` orders communities the way that scan
and reduction prefer them when each sits in its home slot (the reference's
probing after a collision depends on insertion races, and then the smaller
community id wins here).  A vertex keeps at most 1024 distinct neighbour
communities (the reference's table size), taken in order of first appearance
along its row; weights towards later ones are dropped, as the reference drops
them when its table is full.

Sums: the neighbour-community weights are float32 in the reference (float
atomics in an unspecified order); here they are float64 sums rounded to
float32, k_v, Sigma_tot and 2m are float64.  The device adds the same terms in
other orders, so results agree bit for bit whenever these sums are exact (e.g.
dyadic weights) and otherwise differ only when a gain falls within an ulp of
another.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

TABLE_CAP = 1024
M32 = np.uint64(0xFFFFFFFF)


# --------------------------------------------------------------------------- rng.cuh:9-45

def pcg_hash(x):
    """rng.cuh:9-14 (PCG output permutation), vectorised over uint32."""
    x = np.asarray(x, dtype=np.uint64) & M32
    state = (x * np.uint64(747796405) + np.uint64(2891336453)) & M32
    word = (((state >> ((state >> np.uint64(28)) + np.uint64(4))) ^ state) * np.uint64(277803737)) & M32
    return ((word >> np.uint64(22)) ^ word) & M32


def mix4(a, b, c, d):
    h = pcg_hash(a)
    h = pcg_hash(h ^ (np.asarray(b, dtype=np.uint64) & M32))
    h = pcg_hash(h ^ (np.asarray(c, dtype=np.uint64) & M32))
    return pcg_hash(h ^ (np.asarray(d, dtype=np.uint64) & M32))


def _to_unit(h):
    return ((np.asarray(h, dtype=np.uint64) >> np.uint64(8)).astype(np.float32) * np.float32(1.0 / 16777216.0))


def rand_uniform(graph, vertex, level, sweep, seed):
    """rng.cuh:25-31: uniform float32 in [0, 1) from (graph, vertex, level, sweep, seed)."""
    return _to_unit(mix4(graph, vertex, (int(level) << 16) | int(sweep), seed))


def rand_uniform_pair(graph, vertex, candidate, level, sweep, seed):
    """rng.cuh:37-45: per-(vertex, candidate) uniform for Gumbel sampling."""
    s = pcg_hash((np.uint64(int(sweep) << 16)) ^ (np.asarray(candidate, dtype=np.uint64) & M32))
    return _to_unit(mix4(graph, vertex, np.uint64(int(level) << 16) | (s & np.uint64(0xFFFF)), seed))


def _bitrev5(x):
    x = np.asarray(x, dtype=np.int64)
    r = np.zeros_like(x)
    for i in range(5):
        r |= ((x >> i) & 1) << (4 - i)
    return r


def slot_key(c):
    """Preference among equal scores (smaller first): the reference's scan
    order of home slot s = pcg_hash(c) & 1023 -- warp (s>>5)&3 and lane s&31
    through shuffle-down trees, then the thread's slice index s>>7."""
    s = (pcg_hash(c) & np.uint64(1023)).astype(np.int64)
    return (_bitrev5((s >> 5) & 3) << 8) | (_bitrev5(s & 31) << 3) | (s >> 7)


# --------------------------------------------------------------------------- csr.cu

@dataclass
class CSR:
    graphs: int
    seq_len: int
    row_ptr: np.ndarray   # int64 [V+1]
    col: np.ndarray       # int32 [E_sym]
    w: np.ndarray         # float32 [E_sym]
    k_v: np.ndarray       # float64 [V]
    two_m: np.ndarray     # float64 [graphs]

    @property
    def V(self) -> int:
        return self.graphs * self.seq_len

    def rows(self) -> np.ndarray:
        return np.repeat(np.arange(self.V, dtype=np.int64), np.diff(self.row_ptr))


def build_csr(src, dst, w, graphs: int, seq_len: int) -> CSR:
    """csr.cu:20-271: mirror non-self edges, keep self-loops once at twice
    their weight; rows sorted by neighbour id (stable for duplicates)."""
    src = np.asarray(src, np.int64)
    dst = np.asarray(dst, np.int64)
    w = np.asarray(w, np.float32)
    V = graphs * seq_len
    self_loop = src == dst
    s = np.concatenate([src, dst[~self_loop]])
    d = np.concatenate([dst, src[~self_loop]])
    ww = np.concatenate([np.where(self_loop, np.float32(2.0) * w, w), w[~self_loop]]).astype(np.float32)
    order = np.lexsort((d, s))
    s, d, ww = s[order], d[order], ww[order]
    row_ptr = np.zeros(V + 1, np.int64)
    np.cumsum(np.bincount(s, minlength=V), out=row_ptr[1:])
    k_v = np.bincount(s, weights=ww.astype(np.float64), minlength=V)
    two_m = k_v.reshape(graphs, seq_len).sum(axis=1)
    return CSR(graphs, seq_len, row_ptr, d.astype(np.int32), ww, k_v, two_m)


def sigma_tot(csr: CSR, labels: np.ndarray) -> np.ndarray:
    """helpers.cu:18-28: Sigma_tot[c] = sum of k_v over vertices labelled c."""
    ok = labels >= 0
    return np.bincount(labels[ok], weights=csr.k_v[ok], minlength=csr.V)


def _community_sums(csr: CSR, labels: np.ndarray, keep: np.ndarray | None = None):
    """Per (vertex, neighbour community): float64 sum of edge weights, self
    loop excluded, at most TABLE_CAP communities per vertex in order of first
    appearance along the row.  Returns (vertex, community, weight as float32)."""
    rows = csr.rows()
    ok = csr.col != rows
    if keep is not None:
        ok &= keep
    idx = np.nonzero(ok)[0]
    v = rows[idx]
    c = labels[csr.col[idx]].astype(np.int64)
    key = v * csr.V + c
    uniq, first, inv = np.unique(key, return_index=True, return_inverse=True)
    sums = np.bincount(inv, weights=csr.w[idx].astype(np.float64), minlength=uniq.size)
    pv = uniq // csr.V
    # rank of each pair among its vertex's communities by first appearance
    first_pos = idx[first]
    order = np.lexsort((first_pos, pv))
    rank = np.empty(uniq.size, np.int64)
    starts = np.searchsorted(pv[order], pv[order], side="left")
    rank[order] = np.arange(uniq.size) - starts
    kept = rank < TABLE_CAP
    return pv[kept], (uniq % csr.V)[kept], sums[kept].astype(np.float32)


def _pick(v, score, key, c, n, stay_score):
    """Per vertex: the best (score desc, slot key asc, id asc) candidate if it
    beats the stay score (ties go to stay).  Returns chosen community or -1."""
    out = np.full(n, -1, np.int64)
    if v.size == 0:
        return out
    order = np.lexsort((c, key, -score.astype(np.float64), v))
    v_s = v[order]
    firsts = order[np.r_[True, v_s[1:] != v_s[:-1]]]
    win = score[firsts] > stay_score[v[firsts]]
    out[v[firsts][win]] = c[firsts][win]
    return out


# --------------------------------------------------------------------------- local_moving.cu:69-210

def move_gains(csr: CSR, labels: np.ndarray, sig: np.ndarray, resolution: float, keep: np.ndarray | None = None):
    """Modularity gain of moving each vertex to each neighbouring community
    other than its own (local_moving.cu:9-18, 151-158; refinement.cu:237-241):
    dQ = (k_v,new - k_v,old)/m + gamma k_v (Sigma_old - k_v - Sigma_new)/(2 m^2),
    with the neighbour-community weights as float32.  ``keep`` restricts the
    CSR entries (refinement: neighbours in the same parent).  Returns
    (vertex, community, dQ)."""
    V = csr.V
    graph = np.arange(V) // csr.seq_len
    pv, pc, pw = _community_sums(csr, labels, keep)
    old = labels.astype(np.int64)
    k_old = np.zeros(V, np.float32)
    is_old = pc == old[pv]
    k_old[pv[is_old]] = pw[is_old]
    m_g = 0.5 * csr.two_m[graph]
    with np.errstate(divide="ignore", invalid="ignore"):
        inv_m = 1.0 / m_g
        inv_2m2 = 1.0 / (2.0 * m_g * m_g)
    v, c, kn = pv[~is_old], pc[~is_old], pw[~is_old]
    k_v = csr.k_v[v]
    dq = ((kn.astype(np.float64) - k_old[v].astype(np.float64)) * inv_m[v]
          + float(resolution) * k_v * ((sig[old[v]] - k_v) - sig[c]) * inv_2m2[v])
    return v, c, dq


def local_moving_sweep(csr: CSR, labels: np.ndarray, sig: np.ndarray, *, resolution: float, level: int,
                       sweep: int, seed: int, up_down: int) -> tuple[np.ndarray, int]:
    V = csr.V
    graph = np.arange(V) // csr.seq_len
    old = labels.astype(np.int64)
    v, c, dq = move_gains(csr, labels, sig, resolution)
    sel = (c > old[v]).astype(np.int64) == up_down
    v, c, dq = v[sel], c[sel], dq[sel]
    jitter = (rand_uniform(graph, np.arange(V), level, sweep, seed) - np.float32(0.5)) * np.float32(1e-9)
    dq_f = dq.astype(np.float32) + jitter[v]
    choice = _pick(v, dq_f, slot_key(c), c, V, np.zeros(V, np.float32))
    active = (np.diff(csr.row_ptr) > 0) & (csr.two_m[graph] > 0)
    new = np.where(active & (choice >= 0), choice, old).astype(np.int32)
    return new, int((new != labels).sum())


# --------------------------------------------------------------------------- refinement.cu:71-300

def gumbel(u):
    u = np.minimum(np.maximum(np.asarray(u, np.float32), np.float32(1e-7)), np.float32(1.0 - 1e-7))
    return -np.log(-np.log(u))


def refine_propose(csr: CSR, parent: np.ndarray, labels: np.ndarray, sig: np.ndarray, parent_sig: np.ndarray, *,
                   resolution: float, theta: float, boltzmann: bool, level: int, sweep: int, seed: int):
    V = csr.V
    verts = np.arange(V)
    graph = verts // csr.seq_len
    rank = mix4(graph, verts, (int(level) << 16) | int(sweep), seed).astype(np.uint32)
    rows = csr.rows()
    within = parent[csr.col] == parent[rows]
    v, c, dq = move_gains(csr, labels, sig, resolution, within)
    not_self = csr.col != rows
    e_to_s = np.bincount(rows[within & not_self], weights=csr.w[within & not_self].astype(np.float64),
                         minlength=V).astype(np.float32)
    two_m = csr.two_m[graph]
    k_v = csr.k_v
    vol_minus = np.maximum(parent_sig[parent] - k_v, 0.0)
    with np.errstate(divide="ignore", invalid="ignore"):
        bound = float(resolution) * k_v * vol_minus / two_m
    old = labels.astype(np.int64)
    ok = dq >= 0.0
    v, c, dq = v[ok], c[ok], dq[ok]
    t = float(theta) if theta > 0 else 1e-3
    inv_theta = np.float32(1.0) / np.float32(t)
    if boltzmann:
        score = (dq * float(inv_theta)).astype(np.float32) + gumbel(
            rand_uniform_pair(graph[v], v, c, level, sweep, seed))
        stay = gumbel(rand_uniform_pair(graph, verts, old, level, sweep, seed))
    else:
        score = dq.astype(np.float32)
        stay = np.zeros(V, np.float32)
    choice = _pick(v, score, slot_key(c), c, V, stay)
    active = (np.diff(csr.row_ptr) > 0) & (two_m > 0) & ~(e_to_s.astype(np.float64) < bound)
    prop = np.where(active & (choice >= 0), choice, old).astype(np.int32)
    return prop, rank


def refine_commit(csr: CSR, parent: np.ndarray, labels: np.ndarray, prop: np.ndarray, rank: np.ndarray):
    rows = csr.rows()
    u = csr.col.astype(np.int64)
    mover = prop != labels
    r = rank.astype(np.int64)
    beats = (u != rows) & (parent[u] == parent[rows]) & mover[u] & (
        (r[u] > r[rows]) | ((r[u] == r[rows]) & (u > rows)))
    lost = np.bincount(rows[beats], minlength=csr.V) > 0
    commit = mover & ~lost
    return np.where(commit, prop, labels).astype(np.int32), int(commit.sum())


# --------------------------------------------------------------------------- leiden.cu:43-205

def modularity_per_graph(csr: CSR, labels: np.ndarray, resolution: float) -> np.ndarray:
    """helpers.cu:41-118: Q_g = sum_in / 2m - gamma * sum_v k_v Sigma[c_v] / (2m)^2."""
    rows = csr.rows()
    sig = sigma_tot(csr, labels)
    same = labels[csr.col] == labels[rows]
    in_sum = np.bincount(rows[same], weights=csr.w[same].astype(np.float64), minlength=csr.V)
    g = np.arange(csr.V) // csr.seq_len
    two_m = csr.two_m[g]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = in_sum / two_m - float(resolution) * csr.k_v * sig[np.maximum(labels, 0)] / (two_m * two_m)
    q = np.where(two_m > 0, q, 0.0)
    return q.reshape(csr.graphs, csr.seq_len).sum(axis=1)


def batched_leiden(src, dst, w, *, graphs: int, seq_len: int, resolution: float = 1.0, theta: float = 0.01,
                   max_inner_iter: int = 16, seed: int = 0, use_boltzmann: bool = False,
                   return_stages: bool = False):
    """One Leiden level (leiden.cu:43-205): identity start, local moving to
    convergence of both directions, refinement from singletons inside the
    local-moving communities.  Labels are global vertex ids; -1 marks vertices
    without edges."""
    V = graphs * seq_len
    if len(src) == 0:
        lab = np.full(V, -1, np.int32)
        return (lab, np.zeros(graphs)) if not return_stages else (lab, np.zeros(graphs), lab)
    csr = build_csr(src, dst, w, graphs, seq_len)
    cur = np.arange(V, dtype=np.int32)
    up_down, stale = 1, 0
    for sweep in range(max_inner_iter):
        cur, moved = local_moving_sweep(csr, cur, sigma_tot(csr, cur), resolution=resolution, level=0,
                                        sweep=sweep, seed=seed, up_down=up_down)
        if moved == 0:
            up_down ^= 1
            stale += 1
            if stale >= 2:
                break
        else:
            stale = 0
    parent = cur.copy()
    psig = sigma_tot(csr, parent)
    cur = np.arange(V, dtype=np.int32)
    for sweep in range(max_inner_iter):
        prop, rank = refine_propose(csr, parent, cur, sigma_tot(csr, cur), psig, resolution=resolution,
                                    theta=theta, boltzmann=use_boltzmann, level=1, sweep=sweep, seed=seed)
        cur, moved = refine_commit(csr, parent, cur, prop, rank)
        if moved == 0:
            break
    mod = modularity_per_graph(csr, cur, resolution)
    cur = np.where(np.diff(csr.row_ptr) == 0, -1, cur).astype(np.int32)
    if return_stages:
        return cur, mod, np.where(np.diff(csr.row_ptr) == 0, -1, parent).astype(np.int32)
    return cur, mod


# --------------------------------------------------------------------------- aggregate.cu, algorithm.py

def aggregate_coo(src, dst, w, labels, super_vertices: int):
    """aggregate.cu:24-184: relabel both ends, canonical (min, max), sort,
    sum duplicates (float32 sums of the sorted run, in order)."""
    s = np.asarray(labels)[np.asarray(src)].astype(np.int64)
    t = np.asarray(labels)[np.asarray(dst)].astype(np.int64)
    key = np.minimum(s, t) * super_vertices + np.maximum(s, t)
    order = np.argsort(key, kind="stable")
    key, ww = key[order], np.asarray(w, np.float32)[order]
    uniq, start = np.unique(key, return_index=True)
    sums = np.add.reduceat(ww, start) if ww.size else ww
    return (uniq // super_vertices).astype(np.int32), (uniq % super_vertices).astype(np.int32), sums.astype(np.float32)


def densify_per_graph(labels, graphs: int, seq_len: int):
    """algorithm.py:30-48: per-graph rank of each label among the graph's
    distinct labels, offset by g * (max distinct count)."""
    lab = np.asarray(labels).reshape(graphs, seq_len)
    inv, counts = [], []
    for g in range(graphs):
        u, i = np.unique(lab[g], return_inverse=True)
        inv.append(i.astype(np.int32))
        counts.append(u.size)
    width = max(counts)
    dense = np.concatenate([inv[g] + g * width for g in range(graphs)]).astype(np.int32)
    return dense, int(width)


def disjoint_modularity(src, dst, w, labels, resolution: float) -> float:
    """algorithm.py:166-199: Newman modularity of the disjoint union."""
    if len(src) == 0:
        return 0.0
    src = np.asarray(src, np.int64)
    dst = np.asarray(dst, np.int64)
    w64 = np.asarray(w, np.float32).astype(np.float64)
    labels = np.asarray(labels, np.int64)
    k = np.bincount(src, weights=w64, minlength=labels.size) + np.bincount(dst, weights=w64, minlength=labels.size)
    two_m = float(k.sum())
    if two_m <= 0:
        return 0.0
    in_total = 2.0 * float(w64[labels[src] == labels[dst]].sum())
    _, inv = np.unique(labels, return_inverse=True)
    sig = np.bincount(inv, weights=k)
    return in_total / two_m - resolution * float((sig * sig).sum()) / (two_m * two_m)


def run_leiden(src, dst, w, *, graphs: int, seq_len: int, max_level: int = 6, resolution: float = 1.0,
               theta: float = 0.01, max_inner_iter: int = 16, seed: int = 0, use_boltzmann: bool = False):
    """algorithm.py:51-161: levels of (Leiden -> per-graph densify ->
    aggregate), composed back to the original vertices.  Returns
    (vertices with edges, their partition ids, modularity)."""
    V = graphs * seq_len
    lab0, _ = batched_leiden(src, dst, w, graphs=graphs, seq_len=seq_len, resolution=resolution, theta=theta,
                             max_inner_iter=max_inner_iter, seed=seed, use_boltzmann=use_boltzmann)
    isolated = lab0 == -1
    cur = np.where(isolated, np.arange(V, dtype=np.int32), lab0)
    dense, width = densify_per_graph(cur, graphs, seq_len)
    chain = dense
    cs, cd, cw = np.asarray(src), np.asarray(dst), np.asarray(w, np.float32)
    prev = seq_len
    agg = dense
    for level in range(1, max_level):
        if width >= prev:
            break
        cs, cd, cw = aggregate_coo(cs, cd, cw, agg, graphs * width)
        if cs.size == 0:
            break
        lab, _ = batched_leiden(cs, cd, cw, graphs=graphs, seq_len=width, resolution=resolution, theta=theta,
                                max_inner_iter=max_inner_iter, seed=seed + level, use_boltzmann=use_boltzmann)
        lab = np.where(lab == -1, np.arange(graphs * width, dtype=np.int32), lab)
        dense_k, nxt = densify_per_graph(lab, graphs, width)
        chain = dense_k[chain]
        prev, width, agg = width, nxt, dense_k
    mod = disjoint_modularity(src, dst, w, chain, resolution)
    keep = ~isolated
    return np.nonzero(keep)[0], chain[keep].astype(np.int32), mod


# --------------------------------------------------------------------------- partition.py:252-353

def fill_isolated(membership: np.ndarray) -> np.ndarray:
    """partition.py:269-273: -1 entries become singletons numbered after the
    row's largest label, in position order."""
    m = np.asarray(membership, np.int64)
    missing = m == -1
    nxt = m.max(axis=1, keepdims=True) + 1
    return np.where(missing, nxt + np.cumsum(missing, axis=1) - 1, m).astype(np.int32)


def dense_remap(membership: np.ndarray) -> np.ndarray:
    """partition.py:276-286: per row, each label's rank among the row's
    distinct labels."""
    out = np.empty_like(np.asarray(membership), dtype=np.int32)
    for g, row in enumerate(np.asarray(membership)):
        _, inv = np.unique(row, return_inverse=True)
        out[g] = inv
    return out


def partition_labels(src, dst, w, *, graphs: int, seq_len: int, resolution: float, max_inner_iter: int,
                     seed: int):
    """partition_graphs (partition.py:289-353) after build_adjacency: Leiden,
    scatter, isolated fill, dense remap.  Returns (community ids [graphs, S],
    modularity)."""
    if len(src) == 0:
        membership = np.full((graphs, seq_len), -1, np.int32)
        mod = 0.0
    else:
        vertex, labels, mod = run_leiden(src, dst, w, graphs=graphs, seq_len=seq_len, resolution=resolution,
                                         max_inner_iter=max_inner_iter, seed=seed)
        membership = np.full(graphs * seq_len, -1, np.int32)
        membership[vertex] = labels
        membership = membership.reshape(graphs, seq_len)
    return dense_remap(fill_isolated(membership)), mod
