"""The Hugging Face plugin's dispatch (behaviour pinned by the reference's
tests/community_kv/attention/test_adapter.py): registration, prefill through
the edge-exporting kernel with the hand-off to the partitioner, decode after
the partitions are ready, and the minimum prompt length.  CPU only: the
prefill kernel and the CUDA event are replaced by recording fakes."""

from __future__ import annotations

from contextlib import nullcontext
from types import SimpleNamespace

import pytest
import torch

from community_kv_amd.attention import adapter


class _Event:
    def __init__(self, *, enable_timing: bool) -> None:
        assert enable_timing is False
        self.recorded = False

    def record(self) -> None:
        self.recorded = True


class _Runtime:
    def __init__(self) -> None:
        self.config = SimpleNamespace(num_sink=2)
        self.submitted = None
        self.ready = False
        self.decode_runtime = SimpleNamespace(decode=self._decode)

    def submit_prefill_layer(self, **kwargs) -> None:
        self.submitted = kwargs

    def ensure_ready(self) -> None:
        self.ready = True

    def _decode(self, **kwargs) -> torch.Tensor:
        self.decode_kwargs = kwargs
        return torch.tensor([7.0])


def test_register_installs_the_attention_function(monkeypatch):
    import transformers.modeling_utils as modeling_utils

    registry = {}
    monkeypatch.setattr(modeling_utils, "ALL_ATTENTION_FUNCTIONS", registry)
    attention = adapter.CommunityKVAttention(_Runtime())
    assert attention.register() == adapter.ATTENTION_IMPLEMENTATION == "community_kv"
    assert registry["community_kv"] == attention.forward


def test_prefill_exports_edges_and_submits_the_layer(monkeypatch):
    runtime = _Runtime()
    attention = adapter.CommunityKVAttention(runtime)
    query = torch.randn(1, 4, 12, 128)
    key = torch.randn(1, 1, 14, 128)   # the cache holds two rows past the prompt
    output = torch.randn(1, 12, 4, 128)
    scores = torch.randn(1, 4, 12, 8)
    indices = torch.zeros_like(scores, dtype=torch.int32)
    seen = {}

    def fake_prefill(q, k, v, **kwargs):
        seen.update(q=q, k=k, v=v, **kwargs)
        return output, None, None, None, scores, indices

    monkeypatch.setattr(adapter, "prefill_attention_topk", fake_prefill)
    monkeypatch.setattr(torch.cuda, "device", lambda _device: nullcontext())
    monkeypatch.setattr(torch.cuda, "Event", _Event)
    out, weights = attention.forward(SimpleNamespace(layer_idx=3), query, key, torch.randn_like(key), None, 0.125)
    assert out is output and weights is None
    assert seen["q"].shape == (1, 12, 4, 128) and seen["k"].shape == (1, 12, 1, 128)
    assert seen["softmax_scale"] == 0.125 and seen["num_sink"] == 2 and "kappa" not in seen
    assert runtime.submitted["layer_idx"] == 3
    assert runtime.submitted["keys"].shape == (1, 12, 128)
    torch.testing.assert_close(runtime.submitted["topk_indices"], indices[0])
    torch.testing.assert_close(runtime.submitted["topk_scores"], scores[0])
    assert runtime.submitted["completion_event"].recorded


def test_decode_waits_for_partitions_then_dispatches():
    runtime = _Runtime()
    attention = adapter.CommunityKVAttention(runtime)
    key = torch.randn(1, 1, 8, 128)
    out, weights = attention.forward(SimpleNamespace(layer_idx=2), torch.randn(1, 4, 1, 128), key, key, None, 0.5)
    assert runtime.ready and weights is None
    assert out.tolist() == [7.0]
    assert runtime.decode_kwargs["layer_idx"] == 2 and runtime.decode_kwargs["softmax_scale"] == 0.5


def test_prefill_shorter_than_sinks_plus_edges_is_rejected():
    attention = adapter.CommunityKVAttention(_Runtime())
    key = torch.randn(1, 1, 9, 128)
    with pytest.raises(ValueError, match="too short"):
        attention.forward(SimpleNamespace(layer_idx=0), torch.randn(1, 4, 9, 128), key, key, None, 1.0)
