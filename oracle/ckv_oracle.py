"""CPU restatement of CommunityKV's sparse decode step (parity oracle).

TEST INFRASTRUCTURE ONLY.  ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` are the only callers.  The product path
(``community_kv_amd``) never imports this module; it runs the HIP kernels and
fails loudly when they are missing.

Every function restates the reference algorithm named in its docstring
(paths relative to the reference repository root).  Arithmetic that the GPU
path must reproduce bit-for-bit (fp16 centroid scores, nearest-centroid
distances, the online update) is written with numpy float32 operations in the
exact operation order the HIP kernels use; attention itself is computed in
float64 and compared with a tolerance.

Pinning (see tests/test_oracle_*.py):
  * selection / packing / materialisation / update: the reference test
    suite's known answers, transcribed to tests/golden/reference_known_answers.json,
    plus brute-force sorting on small inputs;
  * numerics: numpy / torch conversions and numpy.exp / numpy.log;
  * attention: closed-form softmax in float64 (textbook definition) and a
    dense torch SDPA cross-check;
  * partition fixture builders: reference test known answers;
  * scoring (group max, -inf masking, fp16 rounding), nearest-centroid
    assignment, top-k selection, slot materialisation with the window union
    and the layer-wise centroid sync: tests/test_oracle_pins.py (exact
    rational / float64 brute force, brute-force set construction, the
    reference's materialisation answer, hand-computed sync answers);
  * init_modularity_state (community and total weights of the partition
    fixture): tests/test_oracle_pins.py, against hand graphs (an edge inside
    one community, one across two, a zero-weight edge, several graphs), an
    empty graph and a dense symmetric adjacency built by brute force.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle import numerics as nm

F32 = np.float32
HEAD_DIM = 128
ATTENTION_TILE = 64
KAPPA = 8

PER_QUERY_HEAD = "per_query_head"
QUERY_GROUP = "query_group"
LAYER_WISE = "layer_wise"


# ---------------------------------------------------------------------------
# Partition fixture builders (graph/partition.py)
# ---------------------------------------------------------------------------


def aggregation_mappings(aggregation: str, *, query_heads: int, kv_heads: int):
    """Restates ``aggregation_mappings`` (graph/partition.py:71-94) and
    ``GraphAggregation.retrieval_head_count`` (config.py:16-30)."""
    if aggregation == PER_QUERY_HEAD:
        group = query_heads // kv_heads
        rh = np.arange(query_heads, dtype=np.int32)
        return rh, (rh // group).astype(np.int32)
    if aggregation == QUERY_GROUP:
        rh = np.arange(kv_heads, dtype=np.int32)
        return rh, rh.copy()
    rh = np.arange(kv_heads, dtype=np.int32)
    return np.zeros_like(rh), rh


CENTROID_SUM_BLOCK = 64


def blocked_community_sums(ids, rows, capacity, block=CENTROID_SUM_BLOCK):
    """f32 sum of ``rows`` per community ``ids`` in the state-build order:
    members in ascending position (row) order, in blocks of ``block``; each
    block summed in order from +0, then the block sums added in order from +0.
    (The reference adds with ``scatter_add_``, whose GPU order is unspecified;
    any fixed order is a valid restatement, and for communities of at most
    ``block`` members this is the plain in-order sum.)"""
    ids = np.asarray(ids, np.int64)
    rows = np.asarray(rows, np.float32)
    dim = rows.shape[-1]
    out = np.zeros((capacity, dim), np.float32)
    if ids.size == 0:
        return out
    order = np.argsort(ids, kind="stable")           # by community, ascending position within
    sid = ids[order]
    counts = np.bincount(sid, minlength=capacity)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    rank = np.arange(sid.size) - starts[sid]
    nblk = (counts + block - 1) // block
    blk_first = np.concatenate([[0], np.cumsum(nblk)[:-1]])
    bid = blk_first[sid] + rank // block
    acc = np.zeros((int(nblk.sum()), dim), np.float32)
    u = rank % block
    for j in range(block):
        sel = u == j
        acc[bid[sel]] = (acc[bid[sel]] + rows[order[sel]]).astype(np.float32)
    for k in range(int(nblk.max())):
        has = nblk > k
        out[has] = (out[has] + acc[blk_first[has] + k]).astype(np.float32)
    return out


def compute_centroids(community_ids, community_counts, keys, *, to_graph, to_kv,
                      num_sink, max_decode_tokens, fp8=True):
    """Restates ``compute_centroids`` (graph/partition.py:382-454).

    keys: float32 values ``[Hkv, S, D]``.  Returns (centroids, sizes) where
    centroids are E4M3 codes (fp8=True) or float32 values; the sums follow
    ``blocked_community_sums``.
    """
    community_ids = np.asarray(community_ids)
    graphs, seq_len = community_ids.shape
    active_capacity = int(np.max(community_counts))
    capacity = active_capacity + max_decode_tokens
    dim = keys.shape[-1]
    rheads = len(to_graph)
    sums = np.zeros((rheads, capacity, dim), dtype=np.float32)
    sizes = np.zeros((rheads, capacity), dtype=np.int32)
    for r in range(rheads):
        ids = community_ids[to_graph[r], num_sink:].astype(np.int64)
        src = keys[to_kv[r], num_sink:].astype(np.float32)
        sums[r] = blocked_community_sums(ids, src, capacity)
        np.add.at(sizes[r], ids, 1)
    cent = sums.copy()
    cent[:, :active_capacity] = (
        cent[:, :active_capacity]
        / np.maximum(sizes[:, :active_capacity], 1).astype(np.float32)[..., None]
    ).astype(np.float32)
    cent = np.clip(cent, -nm.E4M3_MAX, nm.E4M3_MAX).astype(np.float32)
    if fp8:
        return nm.f32_to_e4m3(cent), sizes
    return cent, sizes


def build_member_csr(community_ids, community_counts, *, num_sink):
    """Restates ``build_member_csr`` (graph/partition.py:457-492): recency
    descending membership."""
    community_ids = np.asarray(community_ids)
    graphs, seq_len = community_ids.shape
    maxc = int(np.max(community_counts))
    offsets = np.zeros((graphs, maxc + 1), dtype=np.int32)
    positions = np.zeros((graphs, seq_len - num_sink), dtype=np.int32)
    pos = np.arange(num_sink, seq_len, dtype=np.int64)
    for g in range(graphs):
        ids = community_ids[g, num_sink:].astype(np.int64)
        key = ids * seq_len + (seq_len - 1 - pos)
        order = np.argsort(key, kind="stable")
        positions[g] = pos[order]
        counts = np.bincount(ids, minlength=maxc)[:maxc]
        offsets[g, 1:] = np.cumsum(counts)
    return offsets, positions


def build_adjacency(topk_indices, topk_scores, query_positions, *, seq_len, lam):
    """Restates ``build_adjacency`` (graph/partition.py:168-249).

    ``topk_indices`` / ``topk_scores`` ``[graphs, rows, kappa]``; row r of graph
    g is position ``query_positions[g, r]``.  Direct edges (position, column)
    for columns in [0, seq_len), weighted ``score * (lam / 2)``; when lam < 1,
    co-occurrence edges between columns k <= l of a row (both valid) weighted
    ``(score_k * score_l) * (1 - lam)``.  Endpoints are graph * seq_len +
    position, stored as (min, max), coalesced (weights summed in edge order)
    and sorted by (src, dst).  Returns (src, dst, weight) int32/int32/f32."""
    idx = np.asarray(topk_indices, np.int64)
    sc = np.asarray(topk_scores, np.float32)
    graphs, rows, kappa = idx.shape
    total = graphs * seq_len
    off = (np.arange(graphs, dtype=np.int64) * seq_len)[:, None]
    src = np.broadcast_to((np.asarray(query_positions, np.int64) + off)[..., None], idx.shape)
    dst = idx + off[..., None]
    ok = (idx >= 0) & (idx < seq_len)
    srcs, dsts, ws = [src[ok]], [dst[ok]], [(sc[ok] * F32(lam / 2.0)).astype(np.float32)]
    if lam < 1.0:
        r, c = np.triu_indices(kappa)
        ci, cj = idx[..., r], idx[..., c]
        ok2 = (ci >= 0) & (ci < seq_len) & (cj >= 0) & (cj < seq_len)
        srcs.append((ci + off[..., None])[ok2])
        dsts.append((cj + off[..., None])[ok2])
        ws.append(((sc[..., r] * sc[..., c]).astype(np.float32)[ok2] * F32(1.0 - lam)).astype(np.float32))
    s_all, d_all = np.concatenate(srcs), np.concatenate(dsts)
    keys = np.minimum(s_all, d_all) * total + np.maximum(s_all, d_all)
    uniq, inv = np.unique(keys, return_inverse=True)
    w = np.zeros(len(uniq), np.float32)
    np.add.at(w, inv.reshape(-1), np.concatenate(ws))
    return (uniq // total).astype(np.int32), (uniq % total).astype(np.int32), w


def init_modularity_state(community_ids, edge_src, edge_dst, edge_weight, *,
                          community_capacity, seq_len):
    """Restates ``init_modularity_state`` (graph/partition.py:495-535)."""
    graphs = community_ids.shape[0]
    cw = np.zeros((graphs, community_capacity), dtype=np.float32)
    tw = np.zeros((graphs,), dtype=np.float32)
    src = np.asarray(edge_src, dtype=np.int64)
    dst = np.asarray(edge_dst, dtype=np.int64)
    w = np.asarray(edge_weight, dtype=np.float32)
    g = src // seq_len
    sc = community_ids[g, src % seq_len].astype(np.int64)
    dc = community_ids[g, dst % seq_len].astype(np.int64)
    flat = cw.reshape(-1)
    np.add.at(flat, g * community_capacity + sc, w)
    np.add.at(flat, g * community_capacity + dc, w)
    np.add.at(tw, g, (F32(2.0) * w).astype(np.float32))
    return cw, tw


def effective_token_budget(configured_budget, prefill_seq_len, num_sink):
    """Restates ``_effective_token_budget`` (runtime.py:22-34)."""
    available = ((prefill_seq_len + 1) // ATTENTION_TILE) * ATTENTION_TILE
    effective = min(configured_budget, available)
    if effective <= num_sink + 1:
        raise ValueError("prefill sequence is too short for the fixed 64-token decode kernel")
    return effective


# ---------------------------------------------------------------------------
# Decode delta chunks (graph/state.py:64-248)
# ---------------------------------------------------------------------------


@dataclass
class DeltaChunks:
    positions: np.ndarray
    chunk_start: np.ndarray
    chunk_capacity: np.ndarray
    chunk_size: np.ndarray
    chunk_next: np.ndarray
    chunk_previous: np.ndarray
    community_head: np.ndarray
    community_tail: np.ndarray
    community_sizes: np.ndarray
    next_free_chunk: np.ndarray
    next_free_position: np.ndarray

    @classmethod
    def allocate(cls, graph_count, community_capacity, max_decode_tokens):
        """Restates ``DecodeDeltaChunks.allocate`` (graph/state.py:80-130)."""
        cs = (graph_count, max_decode_tokens)
        ts = (graph_count, community_capacity)
        return cls(
            positions=np.full((graph_count, 2 * max_decode_tokens), -1, np.int32),
            chunk_start=np.full(cs, -1, np.int32),
            chunk_capacity=np.zeros(cs, np.int32),
            chunk_size=np.zeros(cs, np.int32),
            chunk_next=np.full(cs, -1, np.int32),
            chunk_previous=np.full(cs, -1, np.int32),
            community_head=np.full(ts, -1, np.int32),
            community_tail=np.full(ts, -1, np.int32),
            community_sizes=np.zeros(ts, np.int32),
            next_free_chunk=np.zeros((graph_count,), np.int32),
            next_free_position=np.zeros((graph_count,), np.int32),
        )

    def copy(self):
        return DeltaChunks(**{k: v.copy() for k, v in self.__dict__.items()})

    def append(self, graph, community, position):
        """Restates ``DecodeDeltaChunks.append`` (graph/state.py:190-225)."""
        tail = int(self.community_tail[graph, community])
        tail_size = int(self.chunk_size[graph, tail]) if tail >= 0 else 0
        tail_cap = int(self.chunk_capacity[graph, tail]) if tail >= 0 else 0
        if tail < 0 or tail_size == tail_cap:
            chunk = int(self.next_free_chunk[graph])
            capacity = 1 if tail < 0 else 2 * tail_cap
            start = int(self.next_free_position[graph])
            if chunk >= self.chunk_start.shape[1]:
                raise RuntimeError("decode-delta chunk capacity exhausted")
            if start + capacity > self.positions.shape[1]:
                raise RuntimeError("decode-delta position capacity exhausted")
            self.next_free_chunk[graph] = chunk + 1
            self.next_free_position[graph] = start + capacity
            self.chunk_start[graph, chunk] = start
            self.chunk_capacity[graph, chunk] = capacity
            self.chunk_previous[graph, chunk] = tail
            if tail < 0:
                self.community_head[graph, community] = chunk
            else:
                self.chunk_next[graph, tail] = chunk
            self.community_tail[graph, community] = chunk
            tail = chunk
            tail_size = 0
        start = int(self.chunk_start[graph, tail])
        self.positions[graph, start + tail_size] = position
        self.chunk_size[graph, tail] = tail_size + 1
        self.community_sizes[graph, community] += 1

    def members(self, graph, community):
        """Restates ``DecodeDeltaChunks.members`` (graph/state.py:227-248): oldest first."""
        size = int(self.community_sizes[graph, community])
        out = []
        chunk = int(self.community_head[graph, community])
        while chunk >= 0 and len(out) < size:
            n = int(self.chunk_size[graph, chunk])
            s = int(self.chunk_start[graph, chunk])
            out.extend(int(p) for p in self.positions[graph, s:s + n])
            chunk = int(self.chunk_next[graph, chunk])
        if len(out) != size:
            raise RuntimeError("decode-delta chunk chain ended early")
        return np.asarray(out, dtype=np.int32)


@dataclass
class LayerState:
    """Decode state of one layer (numpy mirror of MutableGraphState + PrefillCSR)."""

    centroids: np.ndarray          # [R, C, D] uint8 E4M3 codes or float32
    community_sizes: np.ndarray    # [R, C] int32
    community_counts: np.ndarray   # [R] int32
    community_weight: np.ndarray   # [graphs, C] float32
    total_weight: np.ndarray       # [graphs] float32
    token_communities: np.ndarray  # [graphs, S_tc] int32
    deltas: DeltaChunks
    to_graph: np.ndarray
    to_kv: np.ndarray
    member_offsets: np.ndarray     # [graphs, C+1]
    member_positions: np.ndarray   # [graphs, P]
    current_position: np.ndarray   # [graphs]
    fp8: bool = True

    def copy(self):
        kw = {}
        for k, v in self.__dict__.items():
            kw[k] = v.copy() if hasattr(v, "copy") and not isinstance(v, bool) else v
        return LayerState(**kw)

    @property
    def retrieval_heads(self):
        return len(self.to_graph)

    @property
    def community_capacity(self):
        return self.centroids.shape[1]

    def centroid_values(self):
        if self.fp8:
            return nm.e4m3_to_f32(self.centroids)
        return self.centroids.astype(np.float32)


# ---------------------------------------------------------------------------
# Scoring and selection (attention/kernels/centroid_selection.py,
# attention/kernels/_csrc/descriptor_selection.cu)
# ---------------------------------------------------------------------------


def pinned_dot16x8(a, b):
    """fp32 dot over the last axis (128) in the scoring kernel's order.

    Eight lanes each own 16 consecutive dims and accumulate them in order
    (each product rounded to fp32, then added; no FMA); the eight partials are
    combined by the butterfly ((p_j + p_{j+4}), then +2, then +1).
    """
    prod = (a * b).astype(np.float32)
    prod = prod.reshape(prod.shape[:-1] + (8, 16))
    acc = prod[..., 0]
    for i in range(1, 16):
        acc = (acc + prod[..., i]).astype(np.float32)
    s = (acc[..., 0:4] + acc[..., 4:8]).astype(np.float32)
    s = (s[..., 0:2] + s[..., 2:4]).astype(np.float32)
    return (s[..., 0] + s[..., 1]).astype(np.float32)


def pinned_sqdist16x8(k, c):
    d = (k - c).astype(np.float32)
    return pinned_dot16x8(d, d)


def score_centroids(query, state: LayerState, group_size):
    """Restates ``_grouped_centroid_score_kernel`` (centroid_selection.py:32-108):
    scores[r,c] = fp16(max_g q[r*G+g] . centroid[r,c]), -inf when c >= count or
    size <= 0.  query: float32 values of the bf16 (or fp32) query ``[Hq, D]``.
    Returns fp16 bits ``[R, C]``."""
    R, C, D = state.centroids.shape
    cent = state.centroid_values()
    scores = np.full((R, C), np.float32(-np.inf), dtype=np.float32)
    for r in range(R):
        count = int(min(state.community_counts[r], C))
        if count <= 0:
            continue
        q = query[r * group_size:(r + 1) * group_size].astype(np.float32)
        dots = pinned_dot16x8(q[:, None, :], cent[r, None, :count, :])  # [G, count]
        best = dots.max(axis=0)
        ok = state.community_sizes[r, :count] > 0
        scores[r, :count] = np.where(ok, best, np.float32(-np.inf))
    return nm.f32_to_f16_bits(scores)


def nearest_centroid(key, state: LayerState, r):
    """Nearest active non-empty centroid of retrieval head r to ``key`` (float32
    [D]) by squared L2 distance in the pinned order; ties -> lowest id.  Returns
    -1 when no community is eligible."""
    count = int(min(state.community_counts[r], state.community_capacity))
    if count <= 0:
        return -1
    cent = state.centroid_values()[r, :count]
    d = pinned_sqdist16x8(key[None, :].astype(np.float32), cent)
    ok = state.community_sizes[r, :count] > 0
    if not ok.any():
        return -1
    d = np.where(ok, d, np.float32(np.inf))
    best = d[ok].min()
    return int(np.flatnonzero(ok & (d == best))[0])


@dataclass
class Selection:
    communities: list          # descriptor order (reference emission order)
    takes: list
    selected_count: int
    threshold_key: int | None


def weighted_prefix_select(keys, sizes, count, budget):
    """Restates ``_weighted_prefix_select``
    (tests/community_kv/attention/kernels/test_centroid_selection.py:36-66):
    rank by (-key, id) and take communities until the budget is filled, the last
    one truncated."""
    ranked = sorted(
        (-int(keys[i]), i, int(sizes[i])) for i in range(count) if int(sizes[i]) > 0
    )
    remaining = budget
    out = []
    for neg_key, cid, size in ranked:
        if remaining == 0:
            break
        take = min(size, remaining)
        out.append((cid, take, -neg_key))
        remaining -= take
    return out, budget - remaining


def emission_order(prefix, keys):
    """Reorders a prefix selection into the kernel's descriptor order
    (descriptor_selection.cu:342-455): all communities strictly above the
    threshold key in id order, then threshold-key communities in id order."""
    if not prefix:
        return [], []
    thr = prefix[-1][2]
    high = sorted((c, t) for c, t, k in prefix if k > thr)
    equal = sorted((c, t) for c, t, k in prefix if k == thr)
    order = high + equal
    return [c for c, _ in order], [t for _, t in order]


def select_head(score_bits, sizes, count, *, mode, budget, topk=0, max_selected=0):
    """Selection for one retrieval head.

    mode == "budget": reference weighted threshold selection of ``budget``
    member tokens (descriptor_selection.cu:164-455).
    mode == "topk": the ``topk`` best communities by (fp16 key desc, id asc),
    taken whole, in the same emission order, capped at ``max_selected`` tokens
    (the last descriptor truncated to its newest members).
    """
    keys = nm.ordered_fp16_key(score_bits)
    count = int(count)
    if mode == "budget":
        prefix, filled = weighted_prefix_select(keys, sizes, count, budget)
        comms, takes = emission_order(prefix, keys)
        thr = prefix[-1][2] if prefix else None
        return Selection(comms, takes, filled, thr)
    ranked = sorted((-int(keys[i]), i, int(sizes[i])) for i in range(count) if int(sizes[i]) > 0)
    chosen = [(cid, size, -nk) for nk, cid, size in ranked[:topk]]
    comms, takes = emission_order(chosen, keys)
    out_c, out_t, total = [], [], 0
    for c, t in zip(comms, takes):
        if total >= max_selected:
            break
        t = min(t, max_selected - total)
        out_c.append(c)
        out_t.append(t)
        total += t
    thr = chosen[-1][2] if chosen else None
    return Selection(out_c, out_t, total, thr)


def tile_descriptors(takes, tile_count, num_sink):
    """Restates ``tile_descriptor_kernel`` (descriptor_selection.cu:457-487):
    first descriptor whose cumulative end exceeds max(t*64 - num_sink, 0),
    clamped to [0, count-1]."""
    ends = np.cumsum(np.asarray(takes, dtype=np.int64))
    n = len(ends)
    out = np.zeros(tile_count, dtype=np.int32)
    for t in range(tile_count):
        off = max(t * ATTENTION_TILE - num_sink, 0)
        lo = int(np.searchsorted(ends, off, side="right"))
        out[t] = max(0, min(lo, n - 1))
    return out


def community_members_newest_first(state: LayerState, graph, community):
    """Restates ``_materialize_positions`` (tests/community_kv/graph/test_state.py:16-29):
    delta members newest first, then the recency-descending prefill CSR."""
    off = state.member_offsets[graph]
    prefill = state.member_positions[graph, off[community]:off[community + 1]]
    delta = state.deltas.members(graph, community)[::-1]
    return np.concatenate([delta, prefill]).astype(np.int32)


def logical_positions(state: LayerState, r, sel: Selection, *, num_sink, sink_positions,
                      local_window, include_current, slot_capacity):
    """KV positions attended by retrieval head r, in the kernel's slot order:
    [sinks][selected, descriptor order, newest first][window][current], padded
    with -1.  Window slots hold cur-W..cur-1, or -1 where the position is a sink
    or already selected (set union).  Restates the slot mapping of
    ``_direct_segmented_partials_kernel`` (segmented_attention.py:98-282) with
    the window extension."""
    g = int(state.to_graph[r])
    cur = int(state.current_position[g])
    out = [int(p) for p in sink_positions[:num_sink]]
    selected = []
    for c, t in zip(sel.communities, sel.takes):
        members = community_members_newest_first(state, g, c)
        selected.extend(int(p) for p in members[:t])
    out.extend(selected)
    if local_window > 0:
        taken = set(selected) | set(out[:num_sink])
        for i in range(local_window):
            p = cur - local_window + i
            out.append(-1 if (p < 0 or p in taken) else p)
    if include_current:
        out.append(cur)
    if len(out) > slot_capacity:
        raise ValueError("slot capacity too small")
    out.extend([-1] * (slot_capacity - len(out)))
    return np.asarray(out, dtype=np.int32)


# ---------------------------------------------------------------------------
# Attention (segmented_attention.py:283-484) in float64
# ---------------------------------------------------------------------------


def attend(query_rows, keys, values, positions, softmax_scale):
    """Exact softmax attention of ``query_rows`` [G, D] over the rows of
    keys/values [S, D] named by ``positions`` (entries < 0 are skipped).
    Returns (out [G, D] float64, lse [G] float64, scores [G, T] float64 with -inf
    at skipped slots)."""
    pos = np.asarray(positions)
    valid = pos >= 0
    k = keys[np.where(valid, pos, 0)].astype(np.float64)
    v = values[np.where(valid, pos, 0)].astype(np.float64)
    s = (query_rows.astype(np.float64) @ k.T) * float(softmax_scale)
    s = np.where(valid[None, :], s, -np.inf)
    m = s.max(axis=1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(axis=1, keepdims=True)
    out = (p @ v) / l
    lse = (m + np.log(l))[:, 0]
    return out, lse, s


def topk_candidates(scores0, positions, num_sink, kappa=KAPPA):
    """Exact top-kappa of the group-lane-0 scores over non-sink attended slots,
    ordered by (score desc, position asc) -- the packed-key order of
    segmented_attention.py:304-331 and 486-544."""
    pos = np.asarray(positions)
    idx = [i for i in range(len(pos)) if i >= num_sink and pos[i] >= 0]
    ranked = sorted(idx, key=lambda i: (-scores0[i], int(pos[i])))[:kappa]
    sc = [float(scores0[i]) for i in ranked]
    ps = [int(pos[i]) for i in ranked]
    while len(ps) < kappa:
        sc.append(-np.inf)
        ps.append(-1)
    return np.asarray(sc), np.asarray(ps, dtype=np.int32)


# ---------------------------------------------------------------------------
# Online update (segmented_attention.py:546-864, 867-950)
# ---------------------------------------------------------------------------


def _centroid_running_mean(state: LayerState, r, community, key_f32, old_size):
    new_size = old_size + 1
    if old_size > 0:
        old = state.centroid_values()[r, community].astype(np.float32)
        upd = ((old * F32(old_size)).astype(np.float32) + key_f32).astype(np.float32)
        upd = (upd / F32(new_size)).astype(np.float32)
    else:
        upd = key_f32.astype(np.float32)
    if state.fp8:
        state.centroids[r, community] = nm.f32_to_e4m3(upd)
    else:
        state.centroids[r, community] = upd


def _delta_append_guarded(state: LayerState, g, a, cur, valid_position):
    """Delta-chunk append exactly as the fused update kernel performs it
    (segmented_attention.py:719-852).  Returns (chunk_overflow, position_overflow)."""
    d = state.deltas
    chunks_per_graph = d.chunk_start.shape[1]
    position_capacity = d.positions.shape[1]
    delta_size = int(d.community_sizes[g, a])
    old_tail = int(d.community_tail[g, a])
    old_cs = int(d.chunk_size[g, old_tail]) if old_tail >= 0 else 0
    old_cc = int(d.chunk_capacity[g, old_tail]) if old_tail >= 0 else 0
    allocate = old_tail < 0 or old_cs >= old_cc
    free_chunk = int(d.next_free_chunk[g])
    free_pos = int(d.next_free_position[g])
    new_cap = 1 if old_tail < 0 else old_cc * 2
    chunk_ov = allocate and free_chunk >= chunks_per_graph
    pos_ov = allocate and free_pos + new_cap > position_capacity
    alloc_ov = chunk_ov or pos_ov
    chunk = free_chunk if allocate else old_tail
    valid_chunk = (not alloc_ov) and 0 <= chunk < chunks_per_graph
    if allocate and not alloc_ov:
        d.next_free_chunk[g] = free_chunk + 1
        d.next_free_position[g] = free_pos + new_cap
        d.chunk_start[g, free_chunk] = free_pos
        d.chunk_capacity[g, free_chunk] = new_cap
        d.chunk_previous[g, free_chunk] = old_tail
        if old_tail < 0:
            d.community_head[g, a] = free_chunk
        else:
            d.chunk_next[g, old_tail] = free_chunk
        d.community_tail[g, a] = free_chunk
    if valid_chunk and valid_position:
        start = free_pos if allocate else int(d.chunk_start[g, old_tail])
        slot = 0 if allocate else old_cs
        d.positions[g, start + slot] = cur
        d.chunk_size[g, chunk] = slot + 1
        d.community_sizes[g, a] = delta_size + 1
    return chunk_ov, pos_ov


def online_update(state: LayerState, r, *, topk_scores, topk_positions, lse, key_f32, lam,
                  sequence_capacity, assignment="delta_q", nearest=-1):
    """One graph's fused online update, owner retrieval head ``r``.

    assignment="delta_q": restates the modularity-gain rule of
    ``_direct_segmented_reduce_update_kernel`` (segmented_attention.py:546-864);
    the reference test oracle ``_online_assign_and_update``
    (tests/community_kv/graph/test_state.py:32-132) states the same rule.
    assignment="nearest_centroid": the new token joins ``nearest`` (computed by
    :func:`nearest_centroid` before the step); no modularity state changes.

    Float32 arithmetic follows the kernel's operation order.  Returns
    (assigned_out, overflow_bits).
    """
    g = int(state.to_graph[r])
    cap = state.community_capacity
    cur = int(state.current_position[g])
    tc_cap = min(int(sequence_capacity), state.token_communities.shape[1])
    active = int(state.community_counts[r])
    if assignment == "delta_q":
        sc = np.asarray(topk_scores, dtype=np.float32)
        ps = np.asarray(topk_positions, dtype=np.int64)
        valid = (ps >= 0) & (ps < tc_cap)
        lse32 = F32(lse)
        p = np.where(valid, nm.ckv_exp((sc - lse32).astype(np.float32)), F32(0.0)).astype(np.float32)
        half_lam = (F32(lam) * F32(0.5)).astype(np.float32)
        dw = (p * half_lam).astype(np.float32)
        nd = F32(0.0)
        ssum = F32(0.0)
        sq = F32(0.0)
        for i in range(len(p)):
            nd = F32(nd + dw[i])
            ssum = F32(ssum + p[i])
            sq = F32(sq + F32(p[i] * p[i]))
        pair = F32(F32(F32(ssum * ssum) - sq) * F32(F32(0.5) * F32(F32(1.0) - F32(lam))))
        comm = np.where(valid, state.token_communities[g, np.clip(ps, 0, state.token_communities.shape[1] - 1)], -1)
        cand = valid & (comm >= 0) & (comm < active)
        K = len(p)
        cw = np.zeros(K, np.float32)
        leader = np.zeros(K, bool)
        for i in range(K):
            acc = F32(0.0)
            first = K
            for j in range(K):
                if cand[j] and comm[j] == comm[i]:
                    acc = F32(acc + dw[j])
                    first = min(first, j)
            cw[i] = acc
            leader[i] = cand[i] and first == i
        old_total = F32(state.total_weight[g])
        two_m = max(F32(F32(2.0) * old_total), F32(1.0))
        oldw = np.where(cand, state.community_weight[g, np.clip(comm, 0, cap - 1)], F32(0.0)).astype(np.float32)
        dq = np.full(K, -np.inf, np.float32)
        for i in range(K):
            if cand[i] and cw[i] > 0.0:
                dq[i] = F32(cw[i] - F32(F32(nd * oldw[i]) / two_m))
        best = dq.max() if K else -np.inf
        best_comm = min([int(comm[i]) for i in range(K) if cand[i] and dq[i] == best], default=0x7FFFFFFF)
        join = bool(best > 0.0)
        assigned = best_comm if join else active
        comm_ov = assigned >= cap
        if not comm_ov:
            for i in range(K):
                if leader[i]:
                    inc = F32(cw[i] + (nd if (join and comm[i] == assigned) else F32(0.0)))
                    state.community_weight[g, comm[i]] = F32(oldw[i] + inc)
            if not join:
                state.community_weight[g, assigned] = nd
            state.community_counts[r] = active + (0 if join else 1)
            state.total_weight[g] = F32(F32(old_total + nd) + pair)
    else:
        assigned = int(nearest) if nearest >= 0 else active
        comm_ov = assigned >= cap
        if nearest < 0 and not comm_ov:
            state.community_counts[r] = active + 1
    assigned_out = -1 if comm_ov else assigned
    valid_position = 0 <= cur < tc_cap
    chunk_ov = pos_ov = False
    if not comm_ov:
        old_size = int(state.community_sizes[r, assigned])
        state.community_sizes[r, assigned] = old_size + 1
        if valid_position:
            state.token_communities[g, cur] = assigned
            _centroid_running_mean(state, r, assigned, key_f32, old_size)
        chunk_ov, pos_ov = _delta_append_guarded(state, g, assigned, cur, valid_position)
    overflow = int(comm_ov) | (int(chunk_ov) << 1) | (int(pos_ov) << 2) | ((0 if valid_position else 1) << 3)
    if overflow == 0:
        state.current_position[g] = cur + 1
    return assigned_out, overflow


def sync_shared(state: LayerState, assigned, overflow, keys_f32, sequence_capacity):
    """Restates ``_sync_shared_graph_centroids_kernel`` (segmented_attention.py:867-950):
    non-owner retrieval heads apply their graph's assignment to their own table."""
    for r in range(state.retrieval_heads):
        g = int(state.to_graph[r])
        if r == g:
            continue
        c = int(assigned[g])
        valid = int(overflow[g]) == 0 and c >= 0
        cur = int(state.current_position[g]) - 1
        tc_cap = min(int(sequence_capacity), state.token_communities.shape[1])
        if not valid:
            continue
        old = int(state.community_sizes[r, c])
        state.community_sizes[r, c] = old + 1
        if 0 <= cur < tc_cap:
            _centroid_running_mean(state, r, c, keys_f32[int(state.to_kv[r]), cur], old)
        state.community_counts[r] = state.community_counts[g]


# ---------------------------------------------------------------------------
# Whole decode step
# ---------------------------------------------------------------------------


@dataclass
class StepParams:
    group_size: int
    num_sink: int = 10
    token_budget: int = 4096
    mode: str = "budget"            # "budget" | "topk"
    topk_communities: int = 8
    max_selected: int = 0           # slot capacity for topk mode
    local_window: int = 0
    include_current: bool = True
    assignment: str = "delta_q"     # "delta_q" | "nearest_centroid" | "none"
    softmax_scale: float = 1.0 / np.sqrt(128.0)
    lam: float = 0.5

    @property
    def selected_budget(self):
        return self.token_budget - self.num_sink - int(self.include_current)

    @property
    def slot_capacity(self):
        sel = self.selected_budget if self.mode == "budget" else self.max_selected
        n = self.num_sink + sel + self.local_window + int(self.include_current)
        return ((n + ATTENTION_TILE - 1) // ATTENTION_TILE) * ATTENTION_TILE


@dataclass
class StepResult:
    scores: np.ndarray
    selections: list
    positions: np.ndarray
    output: np.ndarray
    lse: np.ndarray
    topk_scores: np.ndarray
    topk_positions: np.ndarray
    nearest: np.ndarray
    assigned: np.ndarray = field(default=None)
    overflow: np.ndarray = field(default=None)


def decode_step(state: LayerState, query, keys, values, params: StepParams, *,
                sink_positions=None, sequence_capacity=None, gpu_topk=None, gpu_lse=None):
    """One full decode-layer transition (decode.py:67-111): score, select,
    attend, then update ``state`` in place.

    query [Hq, D], keys/values [Hkv, S, D] float32 values of the stored
    (bf16/fp32) tensors.  When ``gpu_topk=(scores, positions)`` and ``gpu_lse``
    are given the update consumes them (teacher forcing), so the update can be
    checked bit-exactly against a device run whose attention arithmetic differs
    from float64 in the last bits.
    """
    G = params.group_size
    R = state.retrieval_heads
    if sink_positions is None:
        sink_positions = np.arange(params.num_sink, dtype=np.int32)
    if sequence_capacity is None:
        sequence_capacity = keys.shape[1]
    scores = score_centroids(query, state, G)
    nearest = np.full(R, -1, np.int32)
    if params.assignment == "nearest_centroid":
        for r in range(R):
            g = int(state.to_graph[r])
            cur = int(state.current_position[g])
            if 0 <= cur < keys.shape[1]:
                nearest[r] = nearest_centroid(keys[int(state.to_kv[r]), cur], state, r)
    selections = []
    slots = params.slot_capacity
    positions = np.full((R, slots), -1, np.int32)
    for r in range(R):
        sel = select_head(scores[r], state.community_sizes[r], state.community_counts[r],
                          mode=params.mode, budget=params.selected_budget,
                          topk=params.topk_communities, max_selected=params.max_selected)
        selections.append(sel)
        positions[r] = logical_positions(state, r, sel, num_sink=params.num_sink,
                                         sink_positions=sink_positions,
                                         local_window=params.local_window,
                                         include_current=params.include_current,
                                         slot_capacity=slots)
    Hq = R * G
    out = np.zeros((Hq, keys.shape[-1]))
    lse = np.zeros(Hq)
    tk_s = np.full((R, KAPPA), -np.inf)
    tk_p = np.full((R, KAPPA), -1, np.int32)
    for r in range(R):
        kv = int(state.to_kv[r])
        o, l, s = attend(query[r * G:(r + 1) * G], keys[kv], values[kv], positions[r],
                         params.softmax_scale)
        out[r * G:(r + 1) * G] = o
        lse[r * G:(r + 1) * G] = l
        tk_s[r], tk_p[r] = topk_candidates(s[0], positions[r], params.num_sink)
    res = StepResult(scores, selections, positions, out, lse, tk_s, tk_p, nearest)
    if params.assignment == "none":
        return res
    graphs = len(state.total_weight)
    assigned = np.full(graphs, -1, np.int32)
    overflow = np.zeros(graphs, np.int32)
    for r in range(R):
        g = int(state.to_graph[r])
        if r != g:
            continue
        if gpu_topk is not None:
            sc, ps, l0 = gpu_topk[0][r], gpu_topk[1][r], gpu_lse[r * G]
        else:
            sc, ps, l0 = tk_s[r].astype(np.float32), tk_p[r], np.float32(lse[r * G])
        cur = int(state.current_position[g])
        kv = int(state.to_kv[r])
        key = keys[kv, cur] if 0 <= cur < keys.shape[1] else np.zeros(keys.shape[-1], np.float32)
        assigned[g], overflow[g] = online_update(
            state, r, topk_scores=sc, topk_positions=ps, lse=l0, key_f32=key.astype(np.float32),
            lam=params.lam, sequence_capacity=sequence_capacity,
            assignment=params.assignment, nearest=int(nearest[r]))
    if R != graphs:
        sync_shared(state, assigned, overflow, keys, sequence_capacity)
    res.assigned = assigned
    res.overflow = overflow
    return res
