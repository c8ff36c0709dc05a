"""Hugging Face attention-function plugin (reference: attention/adapter.py:15-91).

``CommunityKVAttention(runtime).register()`` installs ``forward`` under
``"community_kv"`` in ``transformers``' attention registry.  Prefill (query
length > 1) runs the MI355X prefill kernel that also exports each query row's
top-8 attention edges and hands them to the runtime; decode (query length 1)
runs the sparse decode step of the layer.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, Any

import torch

from community_kv_amd.attention.flash_attention import prefill_attention_topk

if TYPE_CHECKING:
    from community_kv_amd.runtime import CommunityKVRuntime

ATTENTION_IMPLEMENTATION = "community_kv"
_TOPK_WIDTH = 8


class CommunityKVAttention:
    """The ``community_kv`` attention function of a Hugging Face model: a
    multi-token call is the prompt (MI355X prefill with top-8 edge export, the
    edges handed to the runtime's partitioner), a single-token call is one
    sparse decode step of the layer."""

    IMPL_NAME = ATTENTION_IMPLEMENTATION

    def __init__(self, runtime: "CommunityKVRuntime") -> None:
        self.runtime = runtime

    def register(self) -> str:
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

        ALL_ATTENTION_FUNCTIONS[self.IMPL_NAME] = self.forward
        return self.IMPL_NAME

    def forward(self, module: torch.nn.Module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                attention_mask: torch.Tensor | None, scaling: float, dropout: float = 0.0,
                **kwargs: Any) -> tuple[torch.Tensor, None]:
        """query [B, Hq, S, D]; key/value [B, Hkv, L, D] (the cache, L >= S).
        Returns ([B, S, Hq, D], None).  The mask and dropout are unused: the
        prefill is causal and the decode step attends the selected slots."""
        layer_idx = int(module.layer_idx)
        scale = float(scaling)
        if query.shape[2] == 1:
            return self._decode_step(layer_idx, query, key, value, scale), None
        return self._prefill(layer_idx, query, key, value, scale), None

    def _decode_step(self, layer_idx: int, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                     scale: float) -> torch.Tensor:
        self.runtime.ensure_ready()  # the partitions of the prompt's layers are installed first
        return self.runtime.decode_runtime.decode(layer_idx=layer_idx, query=query, key=key, value=value,
                                                  softmax_scale=scale)

    def _prefill(self, layer_idx: int, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                 scale: float) -> torch.Tensor:
        sinks = self.runtime.config.num_sink
        prompt = query.shape[2]
        if prompt < sinks + _TOPK_WIDTH:
            raise ValueError(f"CommunityKV prefill is too short to build a graph: {prompt} tokens, "
                             f"need at least {sinks + _TOPK_WIDTH} (sinks + top-{_TOPK_WIDTH})")
        # the kernel takes [B, S, H, D] rows; the cache may already hold more rows than the prompt
        rows = [t[:, :, :prompt, :].transpose(1, 2).contiguous() for t in (query, key, value)]
        out, _lse, _acc, _lse_acc, edge_scores, edge_cols = prefill_attention_topk(
            *rows, softmax_scale=scale, num_sink=sinks)
        # the partitioner starts once this layer's edges exist on the device
        with torch.cuda.device(key.device):
            ready = torch.cuda.Event(enable_timing=False)
            ready.record()
        self.runtime.submit_prefill_layer(layer_idx=layer_idx, topk_indices=edge_cols[0], topk_scores=edge_scores[0],
                                          keys=key[0, :, :prompt], completion_event=ready)
        return out


HuggingFaceAttention = CommunityKVAttention

__all__ = ["ATTENTION_IMPLEMENTATION", "CommunityKVAttention", "HuggingFaceAttention"]
