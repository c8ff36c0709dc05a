"""Seeded synthetic decode-layer fixtures (test and benchmark input generator).

TEST INFRASTRUCTURE: builds the inputs that the BASELINE configurations
describe (Gaussian-mixture keys, community labels, centroids, CSR, modularity
state) as numpy arrays.  The state is assembled with the oracle's restatements
of the reference partition builders (graph/partition.py:382-535), so tests can
hand identical state to the oracle and to the device path.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import ckv_oracle as co
from oracle import numerics as nm


@dataclass
class LayerFixture:
    state: co.LayerState
    query: np.ndarray    # [Hq, D] float32 values (bf16-representable when bf16)
    keys: np.ndarray     # [Hkv, S_cap, D] float32 values
    values: np.ndarray   # [Hkv, S_cap, D]
    prefill_len: int
    dtype: str           # "bf16" | "f32"
    aggregation: str
    query_heads: int
    kv_heads: int
    centers: np.ndarray  # [Hkv, C, D]


def zipf_sizes(rng, count, total, *, exponent=1.1, low=8, high=1024):
    """Community sizes ~ Zipf(exponent) clipped to [low, high], rescaled and
    repaired so they sum to ``total``."""
    raw = rng.zipf(exponent, size=count).astype(np.float64)
    raw = np.clip(raw, low, high)
    sizes = np.maximum(1, np.round(raw * (total / raw.sum()))).astype(np.int64)
    diff = total - int(sizes.sum())
    order = np.argsort(-sizes, kind="stable")
    i = 0
    while diff != 0:
        j = order[i % count]
        step = 1 if diff > 0 else -1
        if sizes[j] + step >= 1:
            sizes[j] += step
            diff -= step
        i += 1
    return sizes


def mixture_labels(rng, graphs, seq_len, num_sink, communities, *, zipf=True):
    """Labels [graphs, seq_len]: the non-sink positions are split into
    communities (Zipf sizes or uniform) at randomly interleaved positions;
    sinks get label 0 (they are excluded from the CSR and centroids)."""
    labels = np.zeros((graphs, seq_len), dtype=np.int32)
    n = seq_len - num_sink
    for g in range(graphs):
        if zipf:
            sizes = zipf_sizes(rng, communities, n)
            lab = np.repeat(np.arange(communities, dtype=np.int32), sizes)
        else:
            lab = rng.integers(0, communities, size=n).astype(np.int32)
            # make ids dense
            _, lab = np.unique(lab, return_inverse=True)
            lab = lab.astype(np.int32)
        rng.shuffle(lab)
        labels[g, num_sink:] = lab
    return labels


def to_dtype(x, dtype):
    x = np.asarray(x, dtype=np.float32)
    return nm.f32_to_bf16(x) if dtype == "bf16" else x


def build_layer(*, seed, query_heads, kv_heads, seq_len, communities, num_sink=10,
                max_decode_tokens=16, aggregation=co.QUERY_GROUP, dtype="bf16",
                fp8=True, zipf=True, key_noise=0.3, query_noise=0.5, lam=0.5,
                extra_kv=None):
    """Builds one decode layer's state plus query/K/V following the
    Gaussian-mixture model of BASELINE config 1/2: centers ~ N(0, I),
    key = center[label] + key_noise * N(0, I), value ~ N(0, I), query = a random
    center of the head + query_noise * N(0, I)."""
    rng = np.random.default_rng(seed)
    D = co.HEAD_DIM
    G = query_heads // kv_heads
    to_graph, to_kv = co.aggregation_mappings(aggregation, query_heads=query_heads,
                                              kv_heads=kv_heads)
    graphs = int(to_graph.max()) + 1
    R = len(to_graph)
    gq = query_heads // R
    s_cap = seq_len + (max_decode_tokens + 1 if extra_kv is None else extra_kv)
    labels = mixture_labels(rng, graphs, seq_len, num_sink, communities, zipf=zipf)
    counts = labels[:, num_sink:].max(axis=1) + 1
    centers = rng.standard_normal((kv_heads, int(counts.max()), D)).astype(np.float32)
    # Each KV head draws keys from the labels of the first graph mapped to it.
    kv_graph = np.zeros(kv_heads, dtype=np.int64)
    for r in range(R):
        kv_graph[to_kv[r]] = to_graph[r]
    keys = np.empty((kv_heads, s_cap, D), dtype=np.float32)
    for h in range(kv_heads):
        lab = labels[kv_graph[h]]
        keys[h, :seq_len] = centers[h, lab] + key_noise * rng.standard_normal((seq_len, D))
        # decode-time keys also follow the mixture
        extra = s_cap - seq_len
        lab_x = rng.integers(0, int(counts[kv_graph[h]]), size=extra)
        keys[h, seq_len:] = centers[h, lab_x] + key_noise * rng.standard_normal((extra, D))
    values = rng.standard_normal((kv_heads, s_cap, D)).astype(np.float32)
    keys = to_dtype(keys, dtype)
    values = to_dtype(values, dtype)
    query = np.empty((query_heads, D), dtype=np.float32)
    for r in range(R):
        h = int(to_kv[r])
        c = int(rng.integers(0, int(counts[to_graph[r]])))
        for j in range(gq):
            query[r * gq + j] = centers[h, c] + query_noise * rng.standard_normal(D)
    query = to_dtype(query, dtype)
    centroids, sizes = co.compute_centroids(labels, counts, keys[:, :seq_len], to_graph=to_graph,
                                            to_kv=to_kv, num_sink=num_sink,
                                            max_decode_tokens=max_decode_tokens, fp8=fp8)
    offsets, positions = co.build_member_csr(labels, counts, num_sink=num_sink)
    cap = centroids.shape[1]
    pad = np.empty((graphs, cap + 1), dtype=np.int32)
    pad[:, :offsets.shape[1]] = offsets
    pad[:, offsets.shape[1]:] = offsets[:, -1:]
    # Synthetic modularity state: each non-sink token has two edges to random
    # members of its community, weight lam/2 * U(0.05, 0.5).
    src, dst, w = [], [], []
    for g in range(graphs):
        lab = labels[g, num_sink:]
        # members of every community in ascending position order (one stable sort)
        order = np.argsort(lab, kind="stable")
        bounds = np.searchsorted(lab[order], np.arange(int(counts[g]) + 1))
        for c in range(int(counts[g])):
            members = order[bounds[c]:bounds[c + 1]] + num_sink
            if len(members) < 2:
                continue
            for _ in range(2):
                partner = rng.permutation(members)
                src.append(g * seq_len + members)
                dst.append(g * seq_len + partner)
                w.append((lam / 2) * rng.uniform(0.05, 0.5, size=len(members)))
    src = np.concatenate(src) if src else np.zeros(0, np.int64)
    dst = np.concatenate(dst) if dst else np.zeros(0, np.int64)
    w = np.concatenate(w).astype(np.float32) if w else np.zeros(0, np.float32)
    cw, tw = co.init_modularity_state(labels, src, dst, w, community_capacity=cap, seq_len=seq_len)
    tc = np.full((graphs, seq_len + max_decode_tokens), -1, dtype=np.int32)
    tc[:, :seq_len] = labels
    state = co.LayerState(
        centroids=centroids,
        community_sizes=sizes,
        community_counts=counts[to_graph].astype(np.int32),
        community_weight=cw,
        total_weight=tw,
        token_communities=tc,
        deltas=co.DeltaChunks.allocate(graphs, cap, max_decode_tokens),
        to_graph=to_graph,
        to_kv=to_kv,
        member_offsets=pad,
        member_positions=positions,
        current_position=np.full((graphs,), seq_len, dtype=np.int32),
        fp8=fp8,
    )
    return LayerFixture(state, query, keys, values, seq_len, dtype, aggregation,
                        query_heads, kv_heads, centers)


def fresh_query(fixture: LayerFixture, rng):
    """A new query drawn like the fixture's (random center + noise)."""
    st = fixture.state
    R = st.retrieval_heads
    gq = fixture.query_heads // R
    q = np.empty_like(fixture.query)
    for r in range(R):
        h = int(st.to_kv[r])
        c = int(rng.integers(0, int(st.community_counts[r])))
        c = min(c, fixture.centers.shape[1] - 1)
        for j in range(gq):
            q[r * gq + j] = fixture.centers[h, c] + 0.5 * rng.standard_normal(co.HEAD_DIM)
    return to_dtype(q, fixture.dtype)
