"""bench.py's host-side accounting, on the CPU: the algorithmic-bytes numerator
of the decode roofline against the per-component figures worked out by hand
for BASELINE config 2 (Qwen3-8B layer: 32 query / 8 KV heads, head dim 128,
512 FP8-centroid communities per KV head, 2,176 attended tokens per head),
the traffic summary parser and the CPU-baseline worker count."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

import bench


def _layer(valid_per_head: int, slot_cap: int, communities: int):
    slots = torch.full((bench.HKV, slot_cap), -1, dtype=torch.int32)
    slots[:, :valid_per_head] = torch.arange(valid_per_head, dtype=torch.int32)
    counts = torch.full((bench.HKV,), communities, dtype=torch.int32)
    layer = SimpleNamespace(workspace=SimpleNamespace(selection=SimpleNamespace(slot_positions=slots)),
                            converted=SimpleNamespace(mutable=SimpleNamespace(community_counts=counts)))
    return {"layer": layer}


def test_algorithmic_bytes_config2_components():
    # hand figures (8 KV heads): K+V rows 8 * 2176 * (2 * 128 * 2 B) = 8,912,896 B;
    # slot table 8 * 2240 * 4 B = 71,680 B; query 32 * 128 * 2 B = 8,192 B;
    # centroid rows + size + fp16 score 8 * 512 * (128 + 4 + 2) B = 548,864 B;
    # output 8,192 B and the update's key row + state, 8 * (256 + 256) B = 4,096 B
    att, step, tokens, cent = bench.algorithmic_bytes([_layer(2176, 2240, 512)])
    assert att == 8_912_896 + 71_680 + 8_192
    assert cent == 548_864
    assert step == att + 548_864 + 8_192 + 4_096
    assert tokens == 2176.0


def test_algorithmic_bytes_averages_layers():
    a1 = bench.algorithmic_bytes([_layer(2176, 2240, 512)])
    a2 = bench.algorithmic_bytes([_layer(1000, 2240, 300)])
    both = bench.algorithmic_bytes([_layer(2176, 2240, 512), _layer(1000, 2240, 300)])
    for x, y, m in zip(a1, a2, both):
        assert m == pytest.approx((x + y) / 2)


def test_profiled_traffic_reads_the_committed_summary():
    t = bench.profiled_traffic()
    assert t is not None and t > 0
    # counter traffic can exceed the algorithmic bytes (re-reads) but not by orders of magnitude
    att, _, _, _ = bench.algorithmic_bytes([_layer(2176, 2240, 512)])
    assert 0.5 * att < t < 3.0 * att


@pytest.mark.parametrize("omp, cpus, want", [("16", 192, 16), ("", 8, 8), ("0", 4, 4), ("64", 8, 8)])
def test_cpu_workers_follow_the_job_share(monkeypatch, omp, cpus, want):
    monkeypatch.setenv("OMP_NUM_THREADS", omp)
    monkeypatch.setattr(bench.os, "cpu_count", lambda: cpus)
    assert bench.cpu_workers() == want
