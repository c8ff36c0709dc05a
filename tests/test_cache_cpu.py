"""Behaviour of the fixed-address KV cache (reference interface:
attention/cache.py:9-121).  Properties checked: K/V must be bf16; prompt
writes go to a host cursor and are bounded by the capacity; after
``enable_device_updates`` writes land at a device cursor without moving the
buffers; the cache-wide controls act on every layer; ``reset`` clears the
contents and both cursors.  CPU only."""

from __future__ import annotations

import pytest
import torch

from community_kv_amd.attention.cache import StaticCache, StaticCacheLayer

HEADS, DIM = 3, 8


def _rows(start: int, count: int) -> tuple[torch.Tensor, torch.Tensor]:
    """K rows carrying their own position (start .. start+count-1); V = -K."""
    pos = torch.arange(start, start + count, dtype=torch.float32)
    k = pos.view(1, 1, count, 1).expand(1, HEADS, count, DIM).to(torch.bfloat16).contiguous()
    return k, -k


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_only_bf16_is_stored(dtype):
    layer = StaticCacheLayer(max_cache_len=6)
    k = torch.zeros(1, HEADS, 2, DIM, dtype=dtype)
    with pytest.raises(TypeError, match="BF16"):
        layer.update(k, k)
    assert layer.get_seq_length() == 0


@pytest.mark.parametrize("chunks", [[6], [1, 2, 3], [4, 2]])
def test_host_cursor_fills_to_capacity_then_refuses(chunks):
    layer = StaticCacheLayer(max_cache_len=6)
    at = 0
    for n in chunks:
        keys, values = layer.update(*_rows(at, n))
        at += n
        assert layer.valid_length == at == layer.get_seq_length()
        assert layer.get_mask_sizes(2) == (min(at + 2, 6), 0)
    assert torch.equal(keys[0, :, :, 0].float(), torch.arange(6.0).expand(HEADS, 6))
    assert torch.equal(values, -keys)
    with pytest.raises(ValueError, match="capacity exceeded"):
        layer.update(*_rows(at, 1))
    assert layer.valid_length == 6


def test_device_cursor_appends_in_place():
    layer = StaticCacheLayer(max_cache_len=8)
    with pytest.raises(RuntimeError):
        layer.enable_device_updates()          # no buffers before the prompt
    keys, values = layer.update(*_rows(0, 3))
    addr = (keys.data_ptr(), values.data_ptr())
    layer.enable_device_updates()
    assert layer.device_updates
    for step in range(3):
        k2, v2 = layer.update(*_rows(3 + step, 1))
        assert (k2.data_ptr(), v2.data_ptr()) == addr
        cursor = layer.get_seq_length()
        assert isinstance(cursor, torch.Tensor) and int(cursor) == 4 + step
    assert layer.valid_length == 3                 # the host cursor lags until it is synced
    assert layer.get_mask_sizes(1) == (8, 0)      # the mask covers the whole buffer
    layer.sync_valid_length()
    assert layer.valid_length == 6
    assert torch.equal(keys[0, 1, :, 0].float(), torch.tensor([0, 1, 2, 3, 4, 5, 0, 0], dtype=torch.float32))


def test_cache_controls_act_on_every_layer():
    cache = StaticCache(num_hidden_layers=3, max_cache_len=5)
    for i in range(3):
        cache.layer(i).update(*_rows(0, i + 1))
    assert [cache.valid_length(i) for i in range(3)] == [1, 2, 3]
    cache.enable_device_updates()
    for i in range(3):
        cache.layer(i).update(*_rows(i + 1, 2))
    cache.sync_valid_lengths()
    assert [cache.valid_length(i) for i in range(3)] == [3, 4, 5]
    cache.reset()
    for i in range(3):
        layer = cache.layer(i)
        assert layer.valid_length == 0 and not layer.device_updates
        assert not layer.keys.any() and not layer.values.any() and int(layer.cumulative_length) == 0
    cache.layer(0).update(*_rows(0, 2))       # host cursor again after the reset
    assert cache.valid_length(0) == 2
