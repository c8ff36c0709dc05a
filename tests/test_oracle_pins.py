"""Pins the oracle functions that the reference test suite's known answers do
not cover: centroid scoring, nearest-centroid assignment, top-k selection,
slot materialisation (logical positions) and the layer-wise centroid sync.

Each check is independent of the oracle's own formula: a float64 / exact
rational brute force, a brute-force set construction, a sort, or a hand
computed answer from the reference kernel's rules
(attention/kernels/centroid_selection.py:32-108, 448-534;
attention/kernels/segmented_attention.py:98-282, 867-950;
tests/community_kv/graph/test_state.py:160-175).  CPU only.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import ckv_oracle as co
from oracle import numerics as nm

D = 128


def _state(centroids_f32, sizes, counts, *, graphs=1, to_graph=None, to_kv=None, seq=64, fp8=True):
    """LayerState with the given centroid values (E4M3-encoded when fp8)."""
    centroids_f32 = np.asarray(centroids_f32, np.float32)
    R, C, _ = centroids_f32.shape
    cent = nm.f32_to_e4m3(centroids_f32) if fp8 else centroids_f32.copy()
    to_graph = np.arange(R, dtype=np.int32) if to_graph is None else np.asarray(to_graph, np.int32)
    to_kv = np.arange(R, dtype=np.int32) if to_kv is None else np.asarray(to_kv, np.int32)
    return co.LayerState(
        centroids=cent, community_sizes=np.asarray(sizes, np.int32).reshape(R, C).copy(),
        community_counts=np.asarray(counts, np.int32).copy(),
        community_weight=np.zeros((graphs, C), np.float32), total_weight=np.zeros(graphs, np.float32),
        token_communities=np.full((graphs, seq), -1, np.int32),
        deltas=co.DeltaChunks.allocate(graphs, C, 8), to_graph=to_graph, to_kv=to_kv,
        member_offsets=np.zeros((graphs, C + 1), np.int32), member_positions=np.zeros((graphs, 1), np.int32),
        current_position=np.zeros(graphs, np.int32), fp8=fp8)


def _exact_dot(q, c):
    return sum(Fraction(float(x)) * Fraction(float(y)) for x, y in zip(q, c))


def _fp16_of_exact(v):
    """fp16 bits of an exactly known real (round to nearest even), via float64
    when that is exact; the inputs below keep every sum exact in float64."""
    f = float(v)
    assert Fraction(f) == v
    return int(np.array([f], np.float64).astype(np.float16).view(np.uint16)[0])


# ---------------------------------------------------------------------------
# score_centroids (centroid_selection.py:32-108)
# ---------------------------------------------------------------------------


def _dyadic(rng, shape, lo=-8, hi=8, scale=0.25):
    """Small dyadic values: every product and partial sum is exact in fp32."""
    return (rng.integers(lo, hi + 1, size=shape) * scale).astype(np.float32)


def test_score_centroids_equals_exact_group_max_with_masking():
    rng = np.random.default_rng(11)
    R, G, C = 3, 4, 9
    cent = _dyadic(rng, (R, C, D), -4, 4, 0.5)  # exact in e4m3
    assert np.array_equal(nm.e4m3_to_f32(nm.f32_to_e4m3(cent)), cent)
    q = _dyadic(rng, (R * G, D), -6, 6, 0.125)
    sizes = rng.integers(0, 5, size=(R, C))
    sizes[0, 2] = 0      # empty community inside the active range
    counts = np.array([C, 6, 0], np.int32)  # head 1: communities 6.. inactive; head 2: none active
    st = _state(cent, sizes, counts)
    got = co.score_centroids(q, st, G)
    neg_inf = int(np.array([-np.inf], np.float16).view(np.uint16)[0])
    for r in range(R):
        for c in range(C):
            if c >= counts[r] or sizes[r, c] <= 0:
                assert got[r, c] == neg_inf, (r, c)
                continue
            best = max(_exact_dot(q[r * G + g], cent[r, c]) for g in range(G))
            assert got[r, c] == _fp16_of_exact(best), (r, c)


def test_score_centroids_uses_every_query_of_the_group():
    # only the last query of the group points at the centroid: a score of query 0 alone would be 0
    cent = np.zeros((1, 2, D), np.float32)
    cent[0, 0, 0] = 1.0
    cent[0, 1, 1] = 2.0
    q = np.zeros((4, D), np.float32)
    q[3, 0] = 3.0
    q[2, 1] = -1.0
    st = _state(cent, [[1, 1]], [2])
    got = co.score_centroids(q, st, 4)
    assert got[0, 0] == _fp16_of_exact(Fraction(3))
    assert got[0, 1] == _fp16_of_exact(Fraction(0))  # max(0, 0, -2, 0)


def test_score_centroids_rounds_to_fp16_and_ties_by_id():
    # 1 + 2^-11 lies halfway between two fp16 values: round to even (1.0); equal
    # fp16 keys then tie-break by community id in the selection
    cent = np.zeros((1, 3, D), np.float32)
    cent[0, :, 0] = 1.0
    q = np.zeros((1, D), np.float32)
    q[0, 0] = np.float32(1.0)
    q[0, 1] = np.float32(2.0 ** -11)
    cent[0, 1, 1] = 1.0          # score 1 + 2^-11 -> 1.0 (even)
    cent[0, 2, 1] = 3.0          # score 1 + 3 * 2^-11 -> 1 + 2^-9 (nearest)
    st = _state(cent, [[1, 1, 1]], [3], fp8=False)
    got = co.score_centroids(q, st, 1)
    vals = got.view(np.float16).astype(np.float64)
    assert vals[0, 0] == 1.0 and vals[0, 1] == 1.0
    assert vals[0, 2] == 1.0 + 2.0 ** -9
    sel = co.select_head(got[0], np.array([1, 1, 1]), 3, mode="budget", budget=2)
    assert sel.communities == [2, 0]  # strictly above the threshold first, then the tie by lowest id


def test_score_centroids_general_inputs_within_one_fp16_ulp():
    rng = np.random.default_rng(5)
    R, G, C = 2, 4, 40
    cent = nm.e4m3_to_f32(nm.f32_to_e4m3(rng.standard_normal((R, C, D)).astype(np.float32)))
    q = nm.f32_to_bf16(rng.standard_normal((R * G, D)).astype(np.float32))
    st = _state(cent, np.ones((R, C)), [C, C])
    got = co.score_centroids(q, st, G).view(np.float16).astype(np.float64)
    ref = np.stack([np.max(q[r * G:(r + 1) * G].astype(np.float64) @ cent[r].T.astype(np.float64), axis=0)
                    for r in range(R)])
    ulp = np.abs(np.spacing(ref.astype(np.float16)).astype(np.float64))
    assert np.all(np.abs(got - ref) <= ulp)


# ---------------------------------------------------------------------------
# nearest_centroid (the build's nearest-centroid assignment)
# ---------------------------------------------------------------------------


def test_nearest_centroid_exact_argmin_masks_and_lowest_id():
    rng = np.random.default_rng(3)
    C = 12
    cent = _dyadic(rng, (1, C, D), -4, 4, 0.5)
    cent[0, 7] = cent[0, 3]                 # tie: 3 and 7 equally near
    key = cent[0, 3].copy()  # exactly centroid 3 (distance 0)
    sizes = np.ones((1, C), np.int32)
    st = _state(cent, sizes, [10])
    assert co.nearest_centroid(key, st, 0) == 3
    # the nearest one is empty: the next nearest active, non-empty community wins
    st.community_sizes[0, 3] = 0
    assert co.nearest_centroid(key, st, 0) == 7
    # communities beyond the active count never win, even when nearer
    key2 = cent[0, 11].copy()
    st2 = _state(cent, sizes, [10])
    d = [float(sum((Fraction(float(a)) - Fraction(float(b))) ** 2 for a, b in zip(key2, cent[0, c])))
         for c in range(10)]
    assert co.nearest_centroid(key2, st2, 0) == int(np.argmin(d))
    # nothing eligible
    st3 = _state(cent, np.zeros((1, C)), [10])
    assert co.nearest_centroid(key, st3, 0) == -1
    st4 = _state(cent, sizes, [0])
    assert co.nearest_centroid(key, st4, 0) == -1


def test_nearest_centroid_matches_float64_argmin_on_random_inputs():
    rng = np.random.default_rng(8)
    for trial in range(20):
        C = int(rng.integers(2, 30))
        cent = nm.e4m3_to_f32(nm.f32_to_e4m3(rng.standard_normal((1, C, D)).astype(np.float32)))
        key = nm.f32_to_bf16(rng.standard_normal(D).astype(np.float32))
        sizes = rng.integers(0, 3, size=(1, C))
        count = int(rng.integers(1, C + 1))
        st = _state(cent, sizes, [count])
        d = ((cent[0, :count].astype(np.float64) - key.astype(np.float64)) ** 2).sum(axis=1)
        d[sizes[0, :count] <= 0] = np.inf
        if not np.isfinite(d).any():
            assert co.nearest_centroid(key, st, 0) == -1
            continue
        order = np.sort(d[np.isfinite(d)])
        if len(order) > 1 and order[1] - order[0] < 1e-4 * (1 + order[0]):
            continue  # near tie: the fp32 order decides
        assert co.nearest_centroid(key, st, 0) == int(np.argmin(d))


# ---------------------------------------------------------------------------
# select_head(mode="topk")
# ---------------------------------------------------------------------------


def test_topk_selection_matches_sort_and_cap():
    rng = np.random.default_rng(21)
    for trial in range(300):
        n = int(rng.integers(1, 30))
        scores = rng.standard_normal(n).astype(np.float32)
        if trial % 2:
            scores = np.round(scores * 2) / 2   # fp16 ties
        sizes = rng.integers(0, 7, size=n).astype(np.int32)
        count = int(rng.integers(1, n + 1))
        topk = int(rng.integers(1, 8))
        cap = int(rng.integers(1, 25))
        bits = nm.f32_to_f16_bits(scores)
        sel = co.select_head(bits, sizes, count, mode="topk", budget=0, topk=topk, max_selected=cap)
        h = scores.astype(np.float16)
        # fp16 total order of the reference's ordered key: -0 ranks below +0
        rank = [(float(h[c]), 0 if np.signbit(h[c]) else 1) for c in range(n)]
        chosen = sorted((c for c in range(count) if sizes[c] > 0), key=lambda c: (-rank[c][0], -rank[c][1], c))[:topk]
        if not chosen:
            assert sel.communities == [] and sel.selected_count == 0
            continue
        thr = min(rank[c] for c in chosen)
        order = sorted(c for c in chosen if rank[c] > thr) + sorted(c for c in chosen if rank[c] == thr)
        expect_c, expect_t, total = [], [], 0
        for c in order:
            if total >= cap:
                break
            t = min(int(sizes[c]), cap - total)
            expect_c.append(c)
            expect_t.append(t)
            total += t
        assert sel.communities == expect_c
        assert sel.takes == expect_t
        assert sel.selected_count == total


# ---------------------------------------------------------------------------
# logical_positions (segmented_attention.py:98-282 + the recent window)
# ---------------------------------------------------------------------------


def _members_brute(offsets, positions, deltas_by_comm, c):
    """Newest first: decode deltas in reverse append order, then the prefill
    CSR row (which is recency-descending)."""
    return list(reversed(deltas_by_comm.get(c, []))) + list(positions[offsets[c]:offsets[c + 1]])


def test_logical_positions_reference_materialisation_answer():
    # the reference's answer (test_state.py:160-175): community 0 has prefill
    # members [9, 0] and decode deltas 10, 11; community 2 contributes one member
    offsets = np.array([[0, 2, 3, 5, 5]], np.int32)
    positions = np.array([[9, 0, 7, 4, 1]], np.int32)
    st = _state(np.zeros((1, 4, D), np.float32), [[4, 1, 2, 0]], [3], seq=16)
    st.member_offsets = offsets
    st.member_positions = positions
    st.deltas = co.DeltaChunks.allocate(1, 4, 8)
    st.deltas.append(0, 0, 10)
    st.deltas.append(0, 0, 11)
    st.current_position[0] = 12
    sel = co.Selection(communities=[0, 2], takes=[4, 1], selected_count=5, threshold_key=None)
    out = co.logical_positions(st, 0, sel, num_sink=0, sink_positions=np.zeros(0, np.int32), local_window=0,
                               include_current=False, slot_capacity=8)
    assert out[:5].tolist() == [11, 10, 9, 0, 4]
    assert out[5:].tolist() == [-1, -1, -1]


def test_logical_positions_layout_matches_brute_force_sets():
    rng = np.random.default_rng(4)
    for trial in range(60):
        seq = 200
        C = int(rng.integers(2, 10))
        ns = int(rng.integers(0, 6))
        cur = int(rng.integers(ns + 20, seq - 1))
        # prefill labels for positions ns..cur-1 (a few recent tokens are decode deltas)
        n_delta = int(rng.integers(0, 6))
        labels = rng.integers(0, C, size=seq)
        prefill_end = cur - n_delta
        offsets = np.zeros(C + 1, np.int32)
        rows = []
        for c in range(C):
            mem = [p for p in range(prefill_end - 1, ns - 1, -1) if labels[p] == c]  # recency-descending
            rows.extend(mem)
            offsets[c + 1] = offsets[c] + len(mem)
        st = _state(np.zeros((1, C, D), np.float32), np.zeros((1, C)), [C], seq=seq)
        st.member_offsets = offsets[None, :]
        st.member_positions = np.asarray(rows if rows else [0], np.int32)[None, :]
        st.deltas = co.DeltaChunks.allocate(1, C, 16)
        deltas = {}
        for p in range(prefill_end, cur):
            c = int(labels[p])
            st.deltas.append(0, c, p)
            deltas.setdefault(c, []).append(p)
        st.current_position[0] = cur
        comms = list(rng.permutation(C)[: int(rng.integers(1, C + 1))])
        takes = []
        for c in comms:
            size = len(_members_brute(offsets, np.asarray(rows, np.int32), deltas, c))
            takes.append(int(rng.integers(0, size + 1)) if size else 0)
        sel = co.Selection(communities=comms, takes=takes, selected_count=sum(takes), threshold_key=None)
        W = int(rng.integers(0, 40))
        sinks = np.arange(ns, dtype=np.int32)
        slots = 64 * ((ns + sum(takes) + W + 1 + 63) // 64)
        out = co.logical_positions(st, 0, sel, num_sink=ns, sink_positions=sinks, local_window=W,
                                   include_current=True, slot_capacity=slots)
        # brute force
        expect = list(range(ns))
        chosen = []
        for c, t in zip(comms, takes):
            chosen.extend(_members_brute(offsets, np.asarray(rows, np.int32), deltas, c)[:t])
        expect.extend(chosen)
        taken = set(chosen) | set(range(ns))
        for p in range(cur - W, cur):
            expect.append(p if (p >= 0 and p not in taken) else -1)
        expect.append(cur)
        expect.extend([-1] * (slots - len(expect)))
        assert out.tolist() == expect, trial
        # every attended position appears once
        att = [p for p in out.tolist() if p >= 0]
        assert len(att) == len(set(att))


# ---------------------------------------------------------------------------
# sync_shared (segmented_attention.py:867-950)
# ---------------------------------------------------------------------------


def _shared_state():
    # LAYER_WISE: three retrieval heads share graph 0 (owner: head 0), each on its own KV head
    C = 4
    cent = np.zeros((3, C, D), np.float32)
    cent[:, 1, :] = 2.0
    cent[:, 2, :] = -1.0
    sizes = np.array([[3, 2, 1, 0], [3, 2, 1, 0], [3, 2, 1, 0]], np.int32)
    st = _state(cent, sizes, [4, 3, 3], to_graph=[0, 0, 0], to_kv=[0, 1, 2], seq=8)
    st.current_position[0] = 5  # after the owner's update: the new token is position 4
    return st


def test_sync_shared_known_answer():
    st = _shared_state()
    keys = np.zeros((3, 8, D), np.float32)
    keys[1, 4, :] = 5.0
    keys[2, 4, :] = -4.0
    co.sync_shared(st, assigned=np.array([1]), overflow=np.array([0]), keys_f32=keys, sequence_capacity=8)
    # head 1: size 2 -> 3, centroid (2 * 2 + 5) / 3 = 3 (exact in e4m3)
    assert st.community_sizes[1].tolist() == [3, 3, 1, 0]
    assert np.all(nm.e4m3_to_f32(st.centroids[1, 1]) == 3.0)
    # head 2: (2 * 2 - 4) / 3 = 0
    assert st.community_sizes[2].tolist() == [3, 3, 1, 0]
    assert np.all(nm.e4m3_to_f32(st.centroids[2, 1]) == 0.0)
    # the owner is untouched, the others copy its community count
    assert st.community_sizes[0].tolist() == [3, 2, 1, 0]
    assert st.community_counts.tolist() == [4, 4, 4]


def test_sync_shared_new_community_takes_the_key():
    st = _shared_state()
    keys = np.zeros((3, 8, D), np.float32)
    keys[1, 4, :] = 1.5
    co.sync_shared(st, assigned=np.array([3]), overflow=np.array([0]), keys_f32=keys, sequence_capacity=8)
    assert st.community_sizes[1, 3] == 1
    assert np.all(nm.e4m3_to_f32(st.centroids[1, 3]) == 1.5)  # old size 0: the key itself


@pytest.mark.parametrize("assigned,overflow", [(-1, 0), (1, 1), (1, 4)])
def test_sync_shared_skips_invalid_assignments(assigned, overflow):
    st = _shared_state()
    before = st.copy()
    keys = np.ones((3, 8, D), np.float32)
    co.sync_shared(st, assigned=np.array([assigned]), overflow=np.array([overflow]), keys_f32=keys,
                   sequence_capacity=8)
    assert np.array_equal(st.community_sizes, before.community_sizes)
    assert np.array_equal(st.centroids, before.centroids)
    assert np.array_equal(st.community_counts, before.community_counts)


def test_sync_shared_position_outside_capacity_updates_size_only():
    st = _shared_state()
    st.current_position[0] = 9  # new token at 8, beyond the sequence capacity
    before = st.copy()
    keys = np.ones((3, 9, D), np.float32)
    co.sync_shared(st, assigned=np.array([1]), overflow=np.array([0]), keys_f32=keys, sequence_capacity=8)
    assert st.community_sizes[1, 1] == before.community_sizes[1, 1] + 1
    assert np.array_equal(st.centroids, before.centroids)


# ---------------------------------------------------------------------------
# init_modularity_state (graph/partition.py:495-535)
# ---------------------------------------------------------------------------


def _dense_degrees(labels, edges, capacity):
    """Community degree sums from a dense symmetric adjacency matrix per graph:
    an edge {u, v} of weight w adds w to A[u, v] and to A[v, u] (a self loop
    therefore adds 2w to A[v, v]), a community's weight is the sum of its
    vertices' rows, and a graph's total is the sum of its matrix (2m in the
    modularity definition).  Hand-built, unrelated to the scatter formula."""
    graphs, seq = labels.shape
    cw = np.zeros((graphs, capacity), np.float64)
    tw = np.zeros(graphs, np.float64)
    for g in range(graphs):
        A = np.zeros((seq, seq), np.float64)
        for (gg, u, v, w) in edges:
            if gg != g:
                continue
            A[u, v] += w
            A[v, u] += w
        deg = A.sum(axis=1)
        for vtx in range(seq):
            cw[g, labels[g, vtx]] += deg[vtx]
        tw[g] = A.sum()
    return cw, tw


def _modularity_case(edges, labels, capacity):
    labels = np.asarray(labels, np.int32)
    seq = labels.shape[1]
    src = np.array([g * seq + u for (g, u, v, w) in edges], np.int64)
    dst = np.array([g * seq + v for (g, u, v, w) in edges], np.int64)
    wts = np.array([w for (g, u, v, w) in edges], np.float32)
    cw, tw = co.init_modularity_state(labels, src, dst, wts, community_capacity=capacity, seq_len=seq)
    want_cw, want_tw = _dense_degrees(labels, edges, capacity)
    return cw, tw, want_cw, want_tw


def test_init_modularity_state_hand_graphs():
    # graph 0: vertices 0,1 in community 0; 2,3 in community 1; 4 in community 2 (isolated)
    # graph 1: vertices 0..2 in community 1; 3,4 in community 0
    labels = [[0, 0, 1, 1, 2], [1, 1, 1, 0, 0]]
    edges = [
        (0, 0, 1, 1.5),    # inside community 0: counted at both endpoints -> +3.0
        (0, 1, 2, 0.25),   # across 0 and 1
        (0, 3, 3, 2.0),    # self loop in community 1 -> +4.0
        (0, 2, 3, 0.0),    # zero weight
        (1, 0, 4, 0.5),    # across 1 and 0
        (1, 2, 1, 0.75),   # inside community 1, destination < source
    ]
    cw, tw, want_cw, want_tw = _modularity_case(edges, labels, capacity=4)
    # the hand answer, written out
    assert cw[0].tolist() == [3.25, 4.25, 0.0, 0.0]
    assert cw[1].tolist() == [0.5, 2.0, 0.0, 0.0]
    assert tw.tolist() == [7.5, 2.5]
    assert np.array_equal(cw.astype(np.float64), want_cw)
    assert np.array_equal(tw.astype(np.float64), want_tw)


def test_init_modularity_state_empty_graph():
    cw, tw = co.init_modularity_state(np.zeros((2, 3), np.int32), np.zeros(0, np.int64), np.zeros(0, np.int64),
                                      np.zeros(0, np.float32), community_capacity=5, seq_len=3)
    assert cw.shape == (2, 5) and tw.shape == (2,)
    assert not cw.any() and not tw.any()


def test_init_modularity_state_random_against_dense_adjacency():
    rng = np.random.default_rng(7)
    graphs, seq, capacity = 3, 24, 6
    labels = rng.integers(0, capacity, size=(graphs, seq))
    edges = []
    for _ in range(120):
        g = int(rng.integers(graphs))
        u, v = (int(x) for x in rng.integers(seq, size=2))
        edges.append((g, u, v, float(rng.integers(0, 16)) / 8.0))  # dyadic: float32 sums are exact
    cw, tw, want_cw, want_tw = _modularity_case(edges, labels, capacity)
    assert np.array_equal(cw.astype(np.float64), want_cw)
    assert np.array_equal(tw.astype(np.float64), want_tw)
    # every community weight is a share of its graph's total
    assert np.allclose(cw.sum(axis=1), tw)
