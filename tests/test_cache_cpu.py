"""The cache's host and device cursors (reference behaviour pinned by
tests/community_kv/attention/test_cache.py): bf16 only, a capacity error,
host-cursor prefill writes, device-cursor writes after enable_device_updates,
and the whole-cache controls.  CPU only."""

from __future__ import annotations

import pytest
import torch

from community_kv_amd.attention.cache import StaticCache, StaticCacheLayer


def _kv(tokens: int, fill: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    k = torch.full((1, 2, tokens, 4), fill, dtype=torch.bfloat16)
    return k, k + 1


def test_layer_host_then_device_cursor():
    layer = StaticCacheLayer(5)
    keys, values = layer.update(*_kv(2))
    assert keys.shape == values.shape == (1, 2, 5, 4)
    assert layer.valid_length == 2 and layer.get_mask_sizes(1) == (3, 0)
    layer.enable_device_updates()
    keys2, _ = layer.update(*_kv(1, 4.0))
    assert keys2.data_ptr() == keys.data_ptr()  # fixed address
    assert int(layer.get_seq_length().item()) == 3
    assert torch.all(keys[0, :, 2] == 4.0) and torch.all(keys[0, :, :2] == 1.0)
    assert layer.get_mask_sizes(1) == (5, 0)
    layer.sync_valid_length()
    assert layer.valid_length == 3


def test_layer_rejects_non_bf16_and_overflow():
    layer = StaticCacheLayer(2)
    with pytest.raises(TypeError, match="BF16"):
        layer.update(torch.zeros((1, 1, 1, 4)), torch.zeros((1, 1, 1, 4)))
    layer.update(*_kv(2))
    with pytest.raises(ValueError, match="capacity exceeded"):
        layer.update(*_kv(1))


def test_cache_switches_and_resets_every_layer():
    cache = StaticCache(num_hidden_layers=2, max_cache_len=4)
    for i in range(2):
        cache.layer(i).update(*_kv(1, float(i + 1)))
    cache.enable_device_updates()
    assert all(cache.layer(i).device_updates for i in range(2))
    cache.sync_valid_lengths()
    assert [cache.valid_length(i) for i in range(2)] == [1, 1]
    cache.reset()
    assert [cache.valid_length(i) for i in range(2)] == [0, 0]
    assert not any(cache.layer(i).device_updates for i in range(2))
