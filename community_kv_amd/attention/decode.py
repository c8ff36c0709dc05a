"""Allocation-free decode-layer transition (reference: attention/decode.py:22-111).

``decode_layer`` keeps the reference signature and return value.  Its HIP
launches (score+select, attention with split merge, online update) read and
mutate the caller's fixed-address tensors; the packed C argument structures are
cached on the workspace and rebuilt only when a tensor address changes, so a
step needs no host synchronisation and can be captured in a HIP graph.
``DecodeRuntime(defer_updates=True)`` instead runs each layer's online update
inside the next layer's selection launch (``DecodeCall.score_select_after``).
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass, field

import torch

from community_kv_amd import _native as nat
from community_kv_amd.attention.kernels import _abi
from community_kv_amd.attention.kernels.centroid_selection import CentroidSelectionWorkspace, score_and_select
from community_kv_amd.attention.kernels.segmented_attention import (
    SegmentedAttentionWorkspace,
    segmented_attention,
)
from community_kv_amd.graph.kernels.online_update import OnlineUpdateWorkspace
from community_kv_amd.graph.state import MutableGraphState, PrefillCSR


@dataclass(slots=True)
class DecodeLayerWorkspace:
    selection: CentroidSelectionWorkspace
    attention: SegmentedAttentionWorkspace
    update: OnlineUpdateWorkspace
    _call_key: tuple | None = field(default=None, repr=False)
    _call: _abi.DecodeCall | None = field(default=None, repr=False)

    @classmethod
    def allocate(cls, *, retrieval_head_count: int, graph_count: int, group_size: int = 4,
                 community_capacity: int, token_budget: int, num_sink: int, dtype: torch.dtype,
                 device: torch.device | str, score_community_counts: Sequence[int] | None = None,
                 score_headroom: int = 0, local_window: int = 0, include_current: bool = True,
                 selection: str = "budget", topk_communities: int = 8, max_selected: int = 0,
                 assignment: str = "delta_q") -> "DecodeLayerWorkspace":
        sel = CentroidSelectionWorkspace.allocate(
            kv_heads=retrieval_head_count, community_capacity=community_capacity, token_budget=token_budget,
            num_sink=num_sink, score_community_counts=score_community_counts, score_headroom=score_headroom,
            device=device, local_window=local_window, include_current=include_current, selection=selection,
            topk_communities=topk_communities, max_selected=max_selected)
        return cls(
            selection=sel,
            attention=SegmentedAttentionWorkspace.allocate(
                kv_heads=retrieval_head_count, group_size=group_size, token_budget=token_budget, dtype=dtype,
                device=device, slot_capacity=sel.slot_capacity),
            update=OnlineUpdateWorkspace.allocate(graph_count=graph_count, device=device, assignment=assignment),
        )

    def call(self, *, query, key, value, csr, state, sink_positions, current_position, softmax_scale,
             lam) -> _abi.DecodeCall:
        """The packed launch arguments for these tensors (cached by address)."""
        cache_key = (query.data_ptr(), query.shape, key.data_ptr(), value.data_ptr(), key.shape, key.stride(),
                     id(csr), id(state), sink_positions.data_ptr(), current_position.data_ptr(),
                     float(softmax_scale), float(lam))
        if self._call is None or self._call_key != cache_key:
            device = nat.require_device(query, key, value, state.centroids, current_position)
            self._call = _abi.DecodeCall(
                _abi.kv_struct(query, key, value), _abi.state_struct(state, current_position),
                _abi.csr_struct(csr), _abi.delta_struct(state.deltas),
                _abi.config_struct(self.selection, group_size=self.attention.group_size,
                                   sink_positions=sink_positions, softmax_scale=softmax_scale, lam=lam,
                                   assignment=self.update.assignment),
                _abi.workspace_struct(self.selection, self.attention, self.update), device,
                # the packed structures hold raw device addresses: keep every tensor they point to alive
                keepalive=(query, key, value, csr, state, sink_positions, current_position))
            self._call_key = cache_key
        return self._call


def decode_layer(*, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, csr: PrefillCSR,
                 state: MutableGraphState, sink_positions: torch.Tensor, current_position: torch.Tensor,
                 softmax_scale: float, lam: float, workspace: DecodeLayerWorkspace):
    """One complete layer transition: select, attend, update.

    Returns (output [Hq,128], lse [Hq], topk_scores [R,8], topk_positions [R,8],
    assigned [graphs]), all workspace tensors updated in place.
    """
    workspace.call(query=query, key=key, value=value, csr=csr, state=state, sink_positions=sink_positions,
                   current_position=current_position, softmax_scale=softmax_scale, lam=lam).decode()
    att = workspace.attention
    return att.output, att.lse, att.topk_scores, att.topk_positions, workspace.update.assigned_communities


__all__ = ["DecodeLayerWorkspace", "decode_layer", "score_and_select", "segmented_attention"]
