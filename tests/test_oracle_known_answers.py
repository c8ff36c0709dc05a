"""Pins the CPU oracle against the reference test suite's known answers.

The expected values come from tests/golden/reference_known_answers.json, which
transcribes the reference repository's own test assertions (each entry names
its source file:line).  These tests exercise the oracle only (no GPU).
"""

from __future__ import annotations

import json
import os
from bisect import bisect_right

import numpy as np
import pytest

from oracle import ckv_oracle as co
from oracle import numerics as nm

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def _f(values):
    return np.asarray([float(v) for v in values], dtype=np.float32)


def _select(scores, sizes, budget, active=None):
    bits = nm.f32_to_f16_bits(_f(scores))
    active = len(scores) if active is None else active
    keys = nm.ordered_fp16_key(bits)
    prefix, filled = co.weighted_prefix_select(keys, np.asarray(sizes), active, budget)
    return [(c, t) for c, t, _ in prefix], filled


def test_ordered_fp16_keys_are_monotonic():
    case = GOLDEN["ordered_fp16_monotonic"]
    keys = nm.ordered_fp16_key(nm.f32_to_f16_bits(_f(case["scores"]))).astype(np.int64)
    assert np.all(keys[1:] >= keys[:-1])


def test_weighted_prefix_truncates_last_community():
    case = GOLDEN["weighted_prefix_truncates_last"]
    sel, filled = _select(case["scores"], case["sizes"], case["budget"])
    assert [list(x) for x in sel] == case["expected"]
    assert filled == case["token_count"]


def test_weighted_prefix_breaks_fp16_ties_by_id():
    case = GOLDEN["weighted_prefix_fp16_ties"]
    assert len(np.unique(nm.f32_to_f16_bits(_f(case["scores"])))) == 1
    sel, _ = _select(case["scores"], case["sizes"], case["budget"])
    assert [c for c, _ in sel] == case["expected_ids"]


def test_weighted_prefix_skips_empty_and_inactive():
    case = GOLDEN["weighted_prefix_zero_size_inactive"]
    sel, _ = _select(case["scores"], case["sizes"], case["budget"], case["active"])
    assert [list(x) for x in sel] == case["expected"]


def test_select_head_matches_brute_force_sort():
    rng = np.random.default_rng(7)
    for trial in range(200):
        n = int(rng.integers(1, 40))
        scores = rng.standard_normal(n).astype(np.float32)
        if trial % 3 == 0:  # force fp16 ties
            scores = np.round(scores * 4) / 4
        sizes = rng.integers(0, 9, size=n).astype(np.int32)
        count = int(rng.integers(1, n + 1))
        budget = int(rng.integers(1, 30))
        bits = nm.f32_to_f16_bits(scores)
        sel = co.select_head(bits, sizes, count, mode="budget", budget=budget)
        # brute force: expand each community into size unit tokens ranked by (-score, id)
        order = sorted((i for i in range(count) if sizes[i] > 0),
                       key=lambda i: (-float(np.float16(scores[i])), i))
        take = {}
        left = budget
        for i in order:
            if left == 0:
                break
            t = min(int(sizes[i]), left)
            take[i] = t
            left -= t
        assert dict(zip(sel.communities, sel.takes)) == take
        assert sel.selected_count == budget - left
        # emission order: strictly-above-threshold ids ascending, then threshold ids ascending
        keys = nm.ordered_fp16_key(bits)
        if sel.communities:
            thr = min(int(keys[c]) for c in sel.communities)
            high = sorted(c for c in sel.communities if keys[c] > thr)
            equal = sorted(c for c in sel.communities if keys[c] == thr)
            assert sel.communities == high + equal
            # only the last descriptor may be truncated
            for c, t in zip(sel.communities[:-1], sel.takes[:-1]):
                assert t == sizes[c]


def _pack(selections, token_budget, num_sink):
    """Restatement of the reference's _pack_segments for the tile table."""
    tiles = token_budget // co.ATTENTION_TILE
    out = []
    for sel in selections:
        takes = [t for _, t in sel]
        out.append(co.tile_descriptors(takes, tiles, num_sink).tolist())
    return out


def test_tile_descriptors_match_reference_packing():
    case = GOLDEN["pack_segments_tile_starts"]
    sels = [[tuple(x) for x in s] for s in case["selections"]]
    assert _pack(sels, case["token_budget"], case["num_sink"]) == case["tile_descriptors"]
    ends = [list(np.cumsum([t for _, t in s])) for s in sels]
    assert [e + [0] * (3 - len(e)) for e in ends] == case["cumulative_ends"]
    case = GOLDEN["pack_segments_singletons"]
    sel = [(c, 1) for c in range(case["count"])]
    assert _pack([sel], case["token_budget"], case["num_sink"]) == case["tile_descriptors"]


def test_tile_descriptors_match_bisect_definition():
    rng = np.random.default_rng(3)
    for _ in range(100):
        takes = list(rng.integers(1, 90, size=int(rng.integers(1, 20))))
        budget = 64 * int(rng.integers(1, 8))
        ns = int(rng.integers(0, 12))
        tiles = co.tile_descriptors(takes, budget // 64, ns)
        ends = list(np.cumsum(takes))
        for t in range(budget // 64):
            off = max(0, t * 64 - ns)
            ref = len(ends) - 1 if off >= ends[-1] else bisect_right(ends, off)
            assert tiles[t] == min(ref, len(ends) - 1)


def test_delta_chunks_append_and_members():
    case = GOLDEN["delta_chunks_append"]
    d = co.DeltaChunks.allocate(case["graph_count"], case["community_capacity"], case["max_decode_tokens"])
    for c, p in case["appends"]:
        d.append(0, c, p)
    for c, expected in case["members"].items():
        assert d.members(0, int(c)).tolist() == expected
    assert d.chunk_capacity[0, :3].tolist() == case["chunk_capacity_prefix"]
    assert int(d.next_free_position[0]) == case["next_free_position"]


def _tiny_state(case_state, *, capacity=None, max_decode=None):
    cap = capacity or case_state["community_capacity"]
    md = max_decode or case_state["max_decode_tokens"]
    dim = case_state["head_dim"]
    cent = np.zeros((1, cap, dim), dtype=np.uint8)
    for row, val in case_state["centroid_rows"].items():
        cent[0, int(row)] = nm.f32_to_e4m3(np.full(dim, val, np.float32))
    sizes = np.zeros((1, cap), np.int32)
    sizes[0, :2] = case_state["community_sizes_prefix"]
    tc = np.full((1, case_state["sequence_capacity"]), -1, np.int32)
    for s, e, v in case_state["token_communities"]:
        tc[0, s:e] = v
    return co.LayerState(
        centroids=cent, community_sizes=sizes,
        community_counts=np.array([case_state["community_counts"]], np.int32),
        community_weight=np.zeros((1, cap), np.float32),
        total_weight=np.array([case_state["total_weight"]], np.float32),
        token_communities=tc, deltas=co.DeltaChunks.allocate(1, cap, md),
        to_graph=np.array([0], np.int32), to_kv=np.array([0], np.int32),
        member_offsets=np.zeros((1, cap + 1), np.int32), member_positions=np.zeros((1, 1), np.int32),
        current_position=np.array([0], np.int32), fp8=True)


def test_materialization_reads_delta_newest_first_then_prefill():
    case = GOLDEN["materialize_prefill_then_delta"]
    cap = case["community_capacity"]
    offsets = np.asarray(case["member_offsets"], np.int32)
    pad = np.concatenate([offsets, np.repeat(offsets[:, -1:], cap + 1 - offsets.shape[1], 1)], 1)
    st = co.LayerState(
        centroids=np.zeros((1, cap, 128), np.uint8), community_sizes=np.zeros((1, cap), np.int32),
        community_counts=np.asarray(case["community_counts"], np.int32),
        community_weight=np.zeros((1, cap), np.float32), total_weight=np.zeros(1, np.float32),
        token_communities=np.zeros((1, 16), np.int32),
        deltas=co.DeltaChunks.allocate(1, cap, case["max_decode_tokens"]),
        to_graph=np.array([0], np.int32), to_kv=np.array([0], np.int32),
        member_offsets=pad, member_positions=np.asarray(case["member_positions"], np.int32),
        current_position=np.array([12], np.int32))
    for c, p in case["delta_appends"]:
        st.deltas.append(0, c, p)
    got = []
    for c, t in case["descriptors"]:
        got.extend(co.community_members_newest_first(st, 0, c)[:t].tolist())
    assert got == case["expected"]


def test_online_update_joins_best_neighbor():
    base = GOLDEN["online_update_state"]
    case = GOLDEN["online_update_join"]
    st = _tiny_state(base)
    st.community_weight[0, :2] = case["community_weight_prefix"]
    st.current_position[0] = case["current_position"]
    w0 = np.float32(st.community_weight[0, 0])
    assigned, ov = co.online_update(
        st, 0, topk_scores=case["topk_scores"], topk_positions=case["topk_positions"],
        lse=case["lse"], key_f32=nm.f32_to_bf16(_f(case["key"])), lam=case["lam"],
        sequence_capacity=base["sequence_capacity"])
    assert assigned == case["assigned"] and ov == 0
    assert int(st.community_counts[0]) == case["community_counts"]
    assert st.community_sizes[0, :2].tolist() == case["community_sizes_prefix"]
    assert st.deltas.members(0, 0).tolist() == case["delta_members_0"]
    expect = nm.e4m3_to_f32(nm.f32_to_e4m3(_f(case["centroid_0"])))
    assert np.array_equal(nm.e4m3_to_f32(st.centroids[0, 0]), expect)
    p = np.exp(np.asarray(case["topk_scores"], np.float64) - case["lse"])
    expected_w0 = float(w0) + (p[0] + p[1]) * 0.25 + p.sum() * 0.25
    assert np.isclose(float(st.community_weight[0, 0]), expected_w0, rtol=1e-5)
    assert int(st.current_position[0]) == case["current_position"] + 1


def test_online_update_creates_singleton():
    base = GOLDEN["online_update_state"]
    case = GOLDEN["online_update_singleton"]
    st = _tiny_state(base)
    st.community_weight[0, :2] = case["community_weight_prefix"]
    st.current_position[0] = case["current_position"]
    assigned, ov = co.online_update(
        st, 0, topk_scores=case["topk_scores"], topk_positions=case["topk_positions"],
        lse=case["lse"], key_f32=nm.f32_to_bf16(_f(case["key"])), lam=case["lam"],
        sequence_capacity=base["sequence_capacity"])
    assert assigned == case["assigned"] and ov == 0
    assert int(st.community_counts[0]) == case["community_counts"]
    assert int(st.community_sizes[0, 2]) == case["size_2"]
    assert nm.e4m3_to_f32(st.centroids[0, 2]).tolist() == case["centroid_2"]
    assert st.deltas.members(0, 2).tolist() == case["delta_members_2"]


def test_online_update_thousands_of_singleton_appends():
    base = GOLDEN["online_update_state"]
    case = GOLDEN["online_update_many_appends"]
    steps = case["steps"]
    st = _tiny_state(base, capacity=steps + 2, max_decode=steps)
    st.community_weight[0, :2] = case["community_weight_prefix"]
    for step in range(steps):
        st.current_position[0] = case["first_position"] + step
        assigned, ov = co.online_update(
            st, 0, topk_scores=[case["topk_score"]], topk_positions=[step], lse=case["lse"],
            key_f32=nm.f32_to_bf16(np.full(4, float(step), np.float32)), lam=case["lam"],
            sequence_capacity=base["sequence_capacity"])
        assert assigned == step + 2 and ov == 0
    assert int(st.community_counts[0]) == steps + 2
    assert int(st.deltas.next_free_chunk[0]) == steps
    assert int(st.deltas.next_free_position[0]) == steps
    assert int(st.community_sizes[0, 2:].sum()) == steps
    assert st.deltas.members(0, steps + 1).tolist() == [case["first_position"] + steps - 1]


def test_online_update_reports_overflow_bits():
    base = GOLDEN["online_update_state"]
    # community capacity overflow: singleton with count == capacity
    st = _tiny_state(base, capacity=2)
    st.community_weight[0, :2] = 100.0
    st.current_position[0] = 30
    a, ov = co.online_update(st, 0, topk_scores=[1.0], topk_positions=[4], lse=1.5,
                             key_f32=np.zeros(4, np.float32), lam=0.5, sequence_capacity=70000)
    assert a == -1 and ov & 1 and int(st.current_position[0]) == 30
    # chunk pool exhaustion
    st = _tiny_state(base, max_decode=1)
    st.community_weight[0, :2] = 100.0
    for step, expect in ((0, 0), (1, 2)):
        st.current_position[0] = 40 + step
        a, ov = co.online_update(st, 0, topk_scores=[1.0], topk_positions=[4], lse=1.5,
                                 key_f32=np.zeros(4, np.float32), lam=0.5, sequence_capacity=70000)
        assert ov == expect
    # invalid current position
    st = _tiny_state(base)
    st.current_position[0] = 70000
    _, ov = co.online_update(st, 0, topk_scores=[1.0], topk_positions=[4], lse=1.5,
                             key_f32=np.zeros(4, np.float32), lam=0.5, sequence_capacity=70000)
    assert ov & 8


def test_member_csr_is_recency_descending():
    case = GOLDEN["member_csr_recency"]
    off, pos = co.build_member_csr(np.asarray(case["ids"]), np.asarray(case["counts"]), num_sink=case["num_sink"])
    assert off.tolist() == case["offsets"] and pos.tolist() == case["positions"]


def test_centroids_exclude_sink_and_reserve_headroom():
    case = GOLDEN["centroids_exclude_sink"]
    keys = np.asarray(case["keys"], np.float32)
    tg, tk = np.array([0], np.int32), np.array([0], np.int32)
    cent, sizes = co.compute_centroids(np.asarray(case["ids"]), np.asarray(case["counts"]), keys,
                                       to_graph=tg, to_kv=tk, num_sink=case["num_sink"],
                                       max_decode_tokens=case["max_decode_tokens"])
    assert list(cent.shape) == case["shape"]
    assert sizes.tolist() == case["sizes"]
    assert nm.e4m3_to_f32(cent[0, :2]).tolist() == case["centroids_prefix"]


def test_centroids_follow_retrieval_mappings():
    case = GOLDEN["centroids_follow_mappings"]
    cent, sizes = co.compute_centroids(
        np.asarray(case["ids"]), np.asarray(case["counts"]), np.asarray(case["keys"], np.float32),
        to_graph=np.asarray(case["to_graph"], np.int32), to_kv=np.asarray(case["to_kv"], np.int32),
        num_sink=case["num_sink"], max_decode_tokens=case["max_decode_tokens"])
    assert sizes[:, :2].tolist() == case["sizes_prefix"]
    assert nm.e4m3_to_f32(cent[:, :2, 0]).tolist() == case["centroids_prefix"]


def test_aggregation_mappings():
    case = GOLDEN["aggregation_mappings"]
    for name in (co.PER_QUERY_HEAD, co.QUERY_GROUP, co.LAYER_WISE):
        g, k = co.aggregation_mappings(name, query_heads=case["query_heads"], kv_heads=case["kv_heads"])
        assert [g.tolist(), k.tolist()] == case[name]


def test_effective_token_budget():
    for budget, seq, sink, expected in GOLDEN["effective_token_budget"]["cases"]:
        assert co.effective_token_budget(budget, seq, sink) == expected
    with pytest.raises(ValueError):
        co.effective_token_budget(4096, 10, 10)


@pytest.mark.parametrize("name", ["adjacency_coalesces", "adjacency_discards_outside"])
def test_adjacency_known_answers(name):
    case = GOLDEN[name]
    src, dst, w = co.build_adjacency(np.asarray(case["indices"]), np.asarray(case["scores"], np.float32),
                                     np.asarray(case["query_positions"]), seq_len=case["seq_len"], lam=case["lam"])
    got = {(int(a), int(b)): float(x) for a, b, x in zip(src, dst, w)}
    assert got == {(a, b): x for a, b, x in case["pairs"]}
