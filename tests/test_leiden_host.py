"""Host logic of the multi-level Leiden driver (community_kv_amd.graph.leiden.
algorithm) with the native module replaced, as the reference's own tests do
(tests/community_kv/graph/leiden/test_algorithm.py:36-105).  CPU only."""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch

from community_kv_amd.graph.leiden import algorithm
from oracle import leiden as L

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def _cpu_densify(labels, G, seq_len):
    dense, width = L.densify_per_graph(labels.numpy(), G, seq_len)
    return torch.from_numpy(dense), width


def _install(monkeypatch, labels):
    calls = []

    class _Module:
        @staticmethod
        def batched_leiden(*args):
            calls.append(args)
            return torch.tensor(labels, dtype=torch.int32), torch.zeros(1, dtype=torch.float64)

        @staticmethod
        def aggregate_coo(*args):
            raise AssertionError("single-level run must not aggregate")

    monkeypatch.setattr(algorithm, "_load_module", lambda: _Module)
    monkeypatch.setattr(algorithm, "_densify_per_graph", _cpu_densify)
    return calls


def test_run_leiden_handles_isolates_and_explicit_parameters(monkeypatch):
    ka = GOLDEN["leiden_isolates"]
    calls = _install(monkeypatch, ka["native_labels"])
    vertex, partition, modularity = algorithm.run_leiden(
        torch.tensor([0], dtype=torch.int32), torch.tensor([1], dtype=torch.int32), torch.ones(1), G=ka["G"],
        seq_len=ka["seq_len"], max_level=ka["max_level"], theta=ka["theta"], max_inner_iter=ka["max_inner_iter"],
        use_boltzmann=ka["use_boltzmann"])
    assert vertex.tolist() == ka["vertex"] and partition.tolist() == ka["partition"]
    assert math.isfinite(modularity)
    assert calls[0][7] == ka["theta"] and calls[0][8] == ka["max_inner_iter"] and calls[0][10] is True


def test_run_leiden_applies_environment_overrides(monkeypatch):
    ka = GOLDEN["leiden_env_overrides"]
    calls = _install(monkeypatch, [0, 0])
    for k, v in ka["env"].items():
        monkeypatch.setenv(k, v)
    algorithm.run_leiden(torch.tensor([0], dtype=torch.int32), torch.tensor([1], dtype=torch.int32), torch.ones(1),
                         G=1, seq_len=2, max_level=1)
    assert calls[0][7] == ka["theta"] and calls[0][8] == ka["max_inner_iter"] and calls[0][10] is True


def test_disjoint_modularity_known_answer():
    ka = GOLDEN["leiden_two_component_modularity"]
    q = algorithm._compute_disjoint_modularity(torch.tensor(ka["src"], dtype=torch.int32),
                                               torch.tensor(ka["dst"], dtype=torch.int32),
                                               torch.tensor(ka["weight"]), torch.tensor(ka["labels"]),
                                               ka["resolution"])
    assert q == pytest.approx(ka["modularity"], abs=1e-9)


def test_native_densify_requires_device_tensors():
    with pytest.raises((RuntimeError, ValueError, TypeError)):
        algorithm._densify_per_graph(torch.tensor(GOLDEN["leiden_densify"]["labels"], dtype=torch.int32), 2, 3)


def test_partition_helpers_match_oracle():
    from community_kv_amd.graph import partition as P

    m = torch.tensor([[5, -1, 5, 2, -1], [-1, -1, 0, 0, 7]], dtype=torch.int32)
    filled = P._fill_isolated_vertices(m)
    assert filled.tolist() == L.fill_isolated(m.numpy()).tolist()
    assert P._dense_remap(filled).tolist() == L.dense_remap(filled.numpy()).tolist()
    idx = torch.arange(4 * 3 * 2, dtype=torch.int32).reshape(4, 3, 2)
    g_idx, _, pos = P._reshape_by_aggregation(idx, idx.float(), aggregation="query_group", num_kv_heads=2,
                                              num_sink=1)
    assert g_idx.shape == (2, 6, 2) and pos[0].tolist() == [2, 3, 4, 2, 3, 4]


def test_partition_runtime_guards():
    """PartitionRuntime (graph/runtime.py:29-176): one job per layer, layer
    range, and offload to another GPU is refused (not part of this build)."""
    from community_kv_amd.config import CommunityKVConfig, PartitionConfig
    from community_kv_amd.graph.runtime import PartitionRuntime

    labels = lambda layer, keys, idx, sc: torch.zeros(1, keys.shape[1], dtype=torch.int32)
    keys = torch.zeros(1, 40, 128)
    idx = torch.zeros(1, 31, 8, dtype=torch.int32)
    sc = torch.ones(1, 31, 8)
    kw = dict(topk_indices=idx, topk_scores=sc, keys=keys, completion_event=None, resolution=1.0,
              max_decode_tokens=2)
    rt = PartitionRuntime(algorithm=CommunityKVConfig(num_sink=2, token_budget=64), scheduling=PartitionConfig(),
                          max_layers=2, label_provider=labels)
    with pytest.raises(ValueError, match="out of range"):
        rt.submit(layer_idx=2, **kw)
    off = PartitionRuntime(algorithm=CommunityKVConfig(), scheduling=PartitionConfig(devices=("cuda:1",)),
                           max_layers=1)
    with pytest.raises(NotImplementedError, match="another GPU"):
        off.submit(layer_idx=0, **kw)
    with pytest.raises(ValueError):
        PartitionRuntime(algorithm=CommunityKVConfig(), scheduling=PartitionConfig(), max_layers=0)
    rt.shutdown()
    off.shutdown()


def test_partition_runtime_device_names_and_failed_job_recovery():
    """A device name without an index means the current GPU; a failed job is
    raised once by reset(), after which the runtime serves new requests."""
    from concurrent.futures import Future

    from community_kv_amd.config import CommunityKVConfig, PartitionConfig
    from community_kv_amd.graph import runtime as grt

    cuda0 = torch.device("cuda", 0)
    assert grt._same_device("cuda", cuda0) == (not torch.cuda.is_available() or torch.cuda.current_device() == 0)
    assert grt._same_device("cuda:0", cuda0)
    assert not grt._same_device("cuda:1", cuda0)
    assert not grt._same_device("cpu", cuda0)
    assert grt._same_device("cpu", torch.device("cpu"))

    rt = grt.PartitionRuntime(algorithm=CommunityKVConfig(), scheduling=PartitionConfig(), max_layers=2)
    failed: Future = Future()
    failed.set_exception(RuntimeError("job failed"))
    done: Future = Future()
    done.set_result(None)
    rt._futures = {0: failed, 1: done}
    with pytest.raises(RuntimeError, match="job failed"):
        rt.reset()
    assert not rt._futures and not rt._results
    rt.reset()  # nothing left to raise
    rt.shutdown()


def test_run_leiden_raises_on_flagged_table_overflow(monkeypatch):
    """The native sweeps mark modularity NaN when a neighbour table overflowed."""

    class _Module:
        @staticmethod
        def batched_leiden(*args):
            return torch.tensor([0, 0], dtype=torch.int32), torch.full((1,), float("nan"), dtype=torch.float64)

    monkeypatch.setattr(algorithm, "_load_module", lambda: _Module)
    monkeypatch.setattr(algorithm, "_densify_per_graph", _cpu_densify)
    with pytest.raises(RuntimeError, match="overflowed"):
        algorithm.run_leiden(torch.tensor([0], dtype=torch.int32), torch.tensor([1], dtype=torch.int32),
                             torch.ones(1), G=1, seq_len=2, max_level=1)
