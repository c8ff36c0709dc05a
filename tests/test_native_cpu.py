"""CPU checks of the native library and the host-side API (no GPU needed).

* libckv_amd.so loads and exports every symbol declared in include/ckv_amd.h;
* the library's scalar numerics (compiled for the host from the same source
  the kernels use) match the oracle's bit for bit;
* host validation, workspace contracts and API surface mirror the reference.
"""

from __future__ import annotations

import ctypes
import json
import os
import re

import numpy as np
import pytest
import torch

from community_kv_amd import _native as nat
from oracle import numerics as nm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_known_answers.json")))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(nat.LIB_PATH):
        nat.build()
    return nat.lib()


def test_library_exports_every_declared_symbol(lib):
    header = open(os.path.join(ROOT, "include", "ckv_amd.h")).read()
    declared = set(re.findall(r"^(?:int|int64_t|size_t|void|const char\*)\s+(ckv_\w+)\(", header, re.M))
    assert declared == set(nat.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.ckv_abi_version() == nat.ABI_VERSION


def _host(lib, op, x, out_dtype):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=out_dtype)
    rc = lib.ckv_host_numerics(op, x.ctypes.data, out.ctypes.data, x.size)
    assert rc == 0
    return out


def _floats(n=300_000, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[np.isfinite(x)]
    special = np.array([0.0, -0.0, 448.0, 464.0, 65504.0, 65520.0, 2**-25, 2**-24, 3 * 2**-26, 2**-10,
                        3 * 2**-11, np.inf, -np.inf, 1.0 + 2**-8, 1.0 + 3 * 2**-9], np.float32)
    return np.concatenate([x, special, (rng.standard_normal(n) * 50).astype(np.float32)])


def test_host_fp16_bf16_e4m3_match_oracle_bitwise(lib):
    x = _floats()
    assert np.array_equal(_host(lib, 2, x, np.uint16), nm.f32_to_f16_bits(x))
    assert np.array_equal(_host(lib, 3, x, np.uint16), nm.bf16_bits(x))
    assert np.array_equal(_host(lib, 4, x, np.uint8), nm.f32_to_e4m3(x))
    codes = np.arange(256, dtype=np.float32)
    got = _host(lib, 5, codes, np.float32)
    ref = nm.e4m3_to_f32(np.arange(256, dtype=np.uint8))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])


def test_host_exp_log_match_oracle_bitwise(lib):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-120, 0, 300_000), rng.uniform(-2, 2, 100_000), rng.uniform(0, 88, 10_000),
                        [0.0, -np.inf, np.inf, -87.3, -86.9, 88.8]]).astype(np.float32)
    assert np.array_equal(_host(lib, 0, x, np.float32).view(np.uint32), nm.ckv_exp(x).view(np.uint32))
    y = np.exp(rng.uniform(0, 80, 300_000)).astype(np.float32)
    y = np.concatenate([y, np.float32([1.0, 2.0, 1.41421356, 1.0000001])])
    assert np.array_equal(_host(lib, 1, y, np.float32).view(np.uint32), nm.ckv_log(y).view(np.uint32))


def test_cpu_tensors_are_rejected_without_fallback():
    from community_kv_amd.attention.kernels.centroid_selection import CentroidSelectionWorkspace, score_and_select

    ws = CentroidSelectionWorkspace.allocate(kv_heads=2, community_capacity=32, token_budget=128, num_sink=10,
                                             device="cpu")
    with pytest.raises(RuntimeError, match="GPU only"):
        score_and_select(query=torch.zeros(8, 128, dtype=torch.bfloat16),
                         centroids=torch.zeros(2, 32, 128, dtype=torch.float8_e4m3fn),
                         community_sizes=torch.ones(2, 32, dtype=torch.int32),
                         community_counts=torch.tensor([8, 12], dtype=torch.int32), workspace=ws)


def test_selection_workspace_contract():
    from community_kv_amd.attention.kernels.centroid_selection import CentroidSelectionWorkspace

    case = GOLDEN["selection_workspace"]
    ws = CentroidSelectionWorkspace.allocate(
        kv_heads=case["kv_heads"], community_capacity=case["community_capacity"],
        token_budget=case["token_budget"], num_sink=case["num_sink"],
        score_community_counts=tuple(case["score_community_counts"]), score_headroom=case["score_headroom"],
        device="cpu")
    assert list(ws.scores.shape) == case["scores_shape"]
    assert ws.score_schedule.tolist() == case["score_schedule"]
    assert ws.selected_budget == case["selected_budget"]
    assert list(ws.packed_segments().tile_descriptors.shape) == case["tile_shape"]
    with pytest.raises(ValueError, match="multiple of 64"):
        CentroidSelectionWorkspace.allocate(kv_heads=1, community_capacity=8, token_budget=96, num_sink=1,
                                            device="cpu")


def test_attention_workspace_contract():
    from community_kv_amd.attention.kernels.segmented_attention import TritonSegmentedAttentionWorkspace

    case = GOLDEN["attention_workspace"]
    ws = TritonSegmentedAttentionWorkspace.allocate(kv_heads=case["kv_heads"], group_size=case["group_size"],
                                                    token_budget=case["token_budget"], dtype=torch.bfloat16,
                                                    device="cpu")
    assert list(ws.partial_max.shape) == case["partial_max"]
    assert list(ws.partial_acc.shape) == case["partial_acc"]
    assert list(ws.partial_topk_packed.shape) == case["partial_topk"]
    assert list(ws.output.shape) == case["output"]
    assert ws.topk_positions.dtype == torch.int32
    for kwargs, message in (({"kv_heads": 0}, "kv_heads"), ({"group_size": 17}, "group_size"),
                            ({"token_budget": 96}, "multiple of 64"), ({"dtype": torch.float16}, "BF16")):
        args = dict(kv_heads=1, group_size=4, token_budget=128, dtype=torch.bfloat16, device="cpu")
        args.update(kwargs)
        with pytest.raises((TypeError, ValueError), match=message):
            TritonSegmentedAttentionWorkspace.allocate(**args)


def test_public_api_matches_reference_surface():
    import community_kv_amd

    assert set(community_kv_amd.__all__) == {
        "ATTENTION_IMPLEMENTATION", "CommunityKVAttention", "CommunityKVConfig", "CommunityKVRuntime",
        "GraphAggregation", "HuggingFaceAttention", "PartitionConfig", "StaticCache", "StaticCacheLayer",
        "leiden_max_iterations", "partition_graphs", "partition_query_groups", "prefill_attention_topk"}
    assert community_kv_amd.ATTENTION_IMPLEMENTATION == "community_kv"
    for name in ("MutableGraphState", "PrefillCSR", "ordered_fp16_keys", "weighted_prefix_select"):
        assert not hasattr(community_kv_amd, name)


def test_effective_budget_and_leiden_iterations():
    from community_kv_amd.graph.partition import leiden_max_iterations
    from community_kv_amd.runtime import _effective_token_budget

    for budget, seq, sink, expected in GOLDEN["effective_token_budget"]["cases"]:
        assert _effective_token_budget(configured_budget=budget, prefill_seq_len=seq, num_sink=sink) == expected
    for length, expected in GOLDEN["leiden_max_iterations"]["cases"]:
        assert leiden_max_iterations(length) == expected


def test_partition_builders_match_reference_known_answers():
    from community_kv_amd.graph.partition import aggregation_mappings, build_member_csr, compute_centroids

    case = GOLDEN["member_csr_recency"]
    off, pos = build_member_csr(torch.tensor(case["ids"], dtype=torch.int32), torch.tensor(case["counts"]),
                                num_sink=case["num_sink"])
    assert off.tolist() == case["offsets"] and pos.tolist() == case["positions"]
    case = GOLDEN["centroids_follow_mappings"]
    cent, sizes = compute_centroids(
        torch.tensor(case["ids"], dtype=torch.int32), torch.tensor(case["counts"]), torch.tensor(case["keys"]),
        retrieval_to_graph=torch.tensor(case["to_graph"], dtype=torch.int32),
        retrieval_to_kv=torch.tensor(case["to_kv"], dtype=torch.int32), num_sink=case["num_sink"],
        max_decode_tokens=case["max_decode_tokens"])
    assert sizes[:, :2].tolist() == case["sizes_prefix"]
    assert cent[:, :2, 0].float().tolist() == case["centroids_prefix"]
    case = GOLDEN["aggregation_mappings"]
    from community_kv_amd import GraphAggregation

    for name in ("per_query_head", "query_group", "layer_wise"):
        g, k = aggregation_mappings(GraphAggregation(name), query_heads=case["query_heads"],
                                    kv_heads=case["kv_heads"], device="cpu")
        assert [g.tolist(), k.tolist()] == case[name]


def test_delta_chunks_host_append_matches_reference():
    from community_kv_amd.graph.state import DecodeDeltaChunks

    case = GOLDEN["delta_chunks_append"]
    d = DecodeDeltaChunks.allocate(graph_count=1, community_capacity=case["community_capacity"],
                                   max_decode_tokens=case["max_decode_tokens"])
    for c, p in case["appends"]:
        d.append(0, c, p)
    for c, expected in case["members"].items():
        assert d.members(0, int(c)).tolist() == expected
    assert d.chunk_capacity[0, :3].tolist() == case["chunk_capacity_prefix"]
    assert int(d.next_free_position[0]) == case["next_free_position"]


def test_config_validation():
    from community_kv_amd import CommunityKVConfig

    with pytest.raises(ValueError):
        CommunityKVConfig(token_budget=100)
    with pytest.raises(ValueError):
        CommunityKVConfig(selection="topk")
    with pytest.raises(ValueError):
        CommunityKVConfig(assignment="kmeans")
    cfg = CommunityKVConfig(aggregation="query_group", local_window=128)
    assert cfg.aggregation.value == "query_group"
