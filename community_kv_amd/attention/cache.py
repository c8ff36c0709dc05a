"""Fixed-address bf16 KV cache for prefill and graph-captured decode.

Reference interface: attention/cache.py:9-121 (``StaticCacheLayer``,
``StaticCache``); its tests (tests/community_kv/attention/test_cache.py) pin the
behaviour: bf16 only, a capacity error on overflow, a host cursor while the
prompt is written and a device cursor once graph decode starts.

Each layer owns one [batch, kv_heads, capacity, head_dim] buffer per K and V,
allocated on the first write and never moved, so kernels and captured graphs
can hold their addresses.  Two cursors mark the end of the written tokens:

* ``valid_length`` - a Python int advanced by prefill writes (variable
  lengths, checked against the capacity on the host);
* ``cumulative_length`` - a one-element int32 tensor on the cache's device.
  After ``enable_device_updates`` every write lands at that device cursor and
  advances it on the device, so a replayed decode step appends where the
  previous replay stopped without a host read.  ``sync_valid_length`` copies
  it back to the host cursor (one synchronising read, outside the step).
"""

from __future__ import annotations

import torch
from transformers.cache_utils import Cache, StaticLayer


def _require_bf16(*tensors: torch.Tensor) -> None:
    bad = [t.dtype for t in tensors if t.dtype != torch.bfloat16]
    if bad:
        raise TypeError(f"the CommunityKV cache stores BF16 K/V only (got {bad[0]})")


class StaticCacheLayer(StaticLayer):
    """One decoder layer's K/V storage with a host and a device write cursor."""

    def __init__(self, max_cache_len: int) -> None:
        super().__init__(max_cache_len=max_cache_len)
        self.valid_length = 0
        self.device_updates = False
        self.cumulative_length = torch.zeros(1, dtype=torch.int32)  # on the host until the buffers exist

    # -- Hugging Face cache-layer protocol ----------------------------------

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        _require_bf16(key_states, value_states)
        super().lazy_initialization(key_states, value_states)  # also moves cumulative_length beside the buffers
        self.cumulative_length.zero_()
        self.valid_length = 0

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args: object,
               **kwargs: object) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        tokens = key_states.shape[-2]
        if self.device_updates:
            self._write_at_device_cursor(key_states, value_states, tokens)
        else:
            self._write_at_host_cursor(key_states, value_states, tokens)
        return self.keys, self.values

    def get_mask_sizes(self, query_length: int, *args: object, **kwargs: object) -> tuple[int, int]:
        # under graph decode the host does not know the length: mask over the whole buffer
        kv_length = self.max_cache_len if self.device_updates else min(self.valid_length + query_length,
                                                                      self.max_cache_len)
        return kv_length, 0

    def get_seq_length(self, *args: object, **kwargs: object) -> int | torch.Tensor:
        if not self.is_initialized:
            return 0
        return self.cumulative_length if self.device_updates else self.valid_length

    def reset(self) -> None:
        if self.is_initialized:
            with torch.inference_mode():
                for buffer in (self.keys, self.values, self.cumulative_length):
                    buffer.zero_()
        self.valid_length = 0
        self.device_updates = False

    # -- cursors -------------------------------------------------------------

    def _write_at_host_cursor(self, key_states: torch.Tensor, value_states: torch.Tensor, tokens: int) -> None:
        start = self.valid_length
        if start + tokens > self.max_cache_len:
            raise ValueError(f"KV cache capacity exceeded: {start + tokens} > {self.max_cache_len}")
        self.keys.narrow(2, start, tokens).copy_(key_states)
        self.values.narrow(2, start, tokens).copy_(value_states)
        self.valid_length = start + tokens
        self.cumulative_length.fill_(self.valid_length)

    def _write_at_device_cursor(self, key_states: torch.Tensor, value_states: torch.Tensor, tokens: int) -> None:
        slots = self.cumulative_length.long() + torch.arange(tokens, device=self.keys.device)
        self.keys.index_copy_(2, slots, key_states)
        self.values.index_copy_(2, slots, value_states)
        self.cumulative_length += tokens

    def enable_device_updates(self) -> None:
        """Switches writes to the device cursor (before capturing a decode step)."""
        if not self.is_initialized:
            raise RuntimeError("the cache layer holds no prefill yet; graph decode needs its buffers")
        with torch.inference_mode():
            self.cumulative_length.fill_(self.valid_length)
        self.device_updates = True

    def sync_valid_length(self) -> None:
        """Reads the device cursor back into ``valid_length``."""
        if self.is_initialized:
            self.valid_length = int(self.cumulative_length.item())


class StaticCache(Cache):
    """``StaticCacheLayer`` per decoder layer, switched and synchronised together."""

    def __init__(self, *, num_hidden_layers: int, max_cache_len: int) -> None:
        super().__init__(layers=[StaticCacheLayer(max_cache_len=max_cache_len) for _ in range(num_hidden_layers)])

    def layer(self, layer_idx: int) -> StaticCacheLayer:
        found = self.layers[layer_idx]
        if isinstance(found, StaticCacheLayer):
            return found
        raise TypeError(f"layer {layer_idx} is a {type(found).__name__}, not a StaticCacheLayer")

    def _each(self):
        return (self.layer(i) for i in range(len(self.layers)))

    def valid_length(self, layer_idx: int) -> int:
        return self.layer(layer_idx).valid_length

    def enable_device_updates(self) -> None:
        for layer in self._each():
            layer.enable_device_updates()

    def sync_valid_lengths(self) -> None:
        for layer in self._each():
            layer.sync_valid_length()


__all__ = ["StaticCache", "StaticCacheLayer"]
