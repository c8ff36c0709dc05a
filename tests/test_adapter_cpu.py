"""Dispatch of the ``community_kv`` attention plugin (reference interface:
attention/adapter.py:15-91).  A call with more than one query row is the
prompt: its rows go to the edge-exporting prefill kernel in [B, S, H, D]
layout, and the layer's edges, keys and a completion event go to the
runtime's partitioner.  A one-row call is a decode step, issued only after
the runtime reports its partitions installed.  Prompts shorter than the sinks
plus one top-8 row are refused.

CPU only: the prefill kernel, the device context and the event are replaced
by stand-ins that append to one shared call log, so the tests can check the
order of the steps as well as their arguments."""

from __future__ import annotations

import contextlib
import types

import pytest
import torch

from community_kv_amd.attention import adapter


class CallLog(list):
    def names(self) -> list[str]:
        return [entry[0] for entry in self]


class RecordingRuntime:
    """The three runtime hooks the plugin uses, each logging its call."""

    def __init__(self, log: CallLog, sinks: int) -> None:
        self.log = log
        self.config = types.SimpleNamespace(num_sink=sinks)
        self.decode_runtime = types.SimpleNamespace(decode=self._decode)

    def submit_prefill_layer(self, **kwargs) -> None:
        self.log.append(("submit", kwargs))

    def ensure_ready(self) -> None:
        self.log.append(("ready", {}))

    def _decode(self, **kwargs) -> torch.Tensor:
        self.log.append(("decode", kwargs))
        return torch.full((1, 1, 2, 16), 3.0)


def _install_fake_device(monkeypatch, log: CallLog, out_rows):
    """Replaces the prefill kernel and the CUDA event with loggers; the fake
    kernel returns a fixed output and edge tensors derived from its inputs."""

    def kernel(q, k, v, **kw):
        log.append(("prefill", dict(q=q.clone(), k=k.clone(), v=v.clone(), **kw)))
        heads = q.shape[2]
        scores = torch.arange(heads * q.shape[1] * 8, dtype=torch.float32).reshape(1, heads, q.shape[1], 8)
        cols = (scores.to(torch.int32) % 5)
        return out_rows, None, None, None, scores, cols

    class LoggedEvent:
        def __init__(self, enable_timing: bool = True) -> None:
            self.timing = enable_timing

        def record(self) -> None:
            log.append(("event", {"timing": self.timing}))

    monkeypatch.setattr(adapter, "prefill_attention_topk", kernel)
    monkeypatch.setattr(torch.cuda, "Event", LoggedEvent)
    monkeypatch.setattr(torch.cuda, "device", lambda _dev: contextlib.nullcontext())


def test_register_uses_the_transformers_registry(monkeypatch):
    import transformers.modeling_utils as mu

    table: dict = {"sdpa": object()}
    monkeypatch.setattr(mu, "ALL_ATTENTION_FUNCTIONS", table)
    plugin = adapter.CommunityKVAttention(RecordingRuntime(CallLog(), sinks=4))
    name = plugin.register()
    assert name == "community_kv" == adapter.ATTENTION_IMPLEMENTATION
    assert table[name] == plugin.forward and "sdpa" in table
    assert adapter.HuggingFaceAttention is adapter.CommunityKVAttention


@pytest.mark.parametrize("sinks,prompt,cache_rows", [(0, 8, 8), (4, 20, 32), (10, 18, 18)])
def test_prompt_goes_to_prefill_then_partitioner(monkeypatch, sinks, prompt, cache_rows):
    log = CallLog()
    plugin = adapter.CommunityKVAttention(RecordingRuntime(log, sinks))
    gen = torch.Generator().manual_seed(prompt)
    q = torch.randn(1, 6, prompt, 16, generator=gen)           # 6 query heads
    k = torch.randn(1, 2, cache_rows, 16, generator=gen)       # 2 KV heads, cache may run past the prompt
    v = torch.randn(1, 2, cache_rows, 16, generator=gen)
    out_rows = torch.zeros(1, prompt, 6, 16)
    _install_fake_device(monkeypatch, log, out_rows)

    out, attn = plugin.forward(types.SimpleNamespace(layer_idx=5), q, k, v, torch.ones(1), 0.25, dropout=0.0)

    assert out is out_rows and attn is None
    assert log.names() == ["prefill", "event", "submit"]   # edges exist before the event, event before the hand-off
    call = log[0][1]
    assert torch.equal(call["q"], q.transpose(1, 2))        # [B, S, H, D] rows
    assert torch.equal(call["k"], k[:, :, :prompt].transpose(1, 2))
    assert torch.equal(call["v"], v[:, :, :prompt].transpose(1, 2))
    assert call["softmax_scale"] == 0.25 and call["num_sink"] == sinks
    assert log[1][1] == {"timing": False}
    handed = log[2][1]
    assert handed["layer_idx"] == 5
    assert torch.equal(handed["keys"], k[0, :, :prompt])
    assert handed["topk_scores"].shape == (6, prompt, 8) and handed["topk_indices"].dtype == torch.int32
    assert handed["completion_event"].timing is False


@pytest.mark.parametrize("sinks", [0, 3])
def test_shortest_prompt_is_sinks_plus_eight(monkeypatch, sinks):
    log = CallLog()
    plugin = adapter.CommunityKVAttention(RecordingRuntime(log, sinks))
    _install_fake_device(monkeypatch, log, torch.zeros(1))
    layer = types.SimpleNamespace(layer_idx=0)
    short = sinks + 7
    x = torch.zeros(1, 2, short, 16)
    with pytest.raises(ValueError, match="too short"):
        plugin.forward(layer, x, x[:, :1], x[:, :1], None, 1.0)
    assert log == []                                          # nothing launched for a refused prompt
    x = torch.zeros(1, 2, short + 1, 16)
    plugin.forward(layer, x, x[:, :1], x[:, :1], None, 1.0)
    assert log.names() == ["prefill", "event", "submit"]


def test_single_row_waits_for_partitions_then_decodes():
    log = CallLog()
    plugin = adapter.CommunityKVAttention(RecordingRuntime(log, sinks=1))
    q = torch.randn(1, 2, 1, 16)
    kv = torch.randn(1, 1, 40, 16)
    out, attn = plugin.forward(types.SimpleNamespace(layer_idx=11), q, kv, kv + 1, None, 0.5)
    assert attn is None and torch.all(out == 3.0)
    assert log.names() == ["ready", "decode"]
    args = log[1][1]
    assert args["layer_idx"] == 11 and args["softmax_scale"] == 0.5
    assert args["query"] is q and args["key"] is kv
    assert torch.equal(args["value"], kv + 1)
