"""Packs the host-side dataclasses into the C structures of include/ckv_amd.h.

A :class:`DecodeCall` holds one fully-packed argument set; callers that keep
their tensors at fixed addresses (the decode runtime, benchmarks, graph
capture) build it once and relaunch it every step.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from community_kv_amd import _native as nat


def kv_struct(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> nat.KvCache:
    """query [Hq, 128]; key/value [Hkv, S, 128] (any head/token strides, unit dim stride)."""
    if query.ndim != 2 or query.shape[1] != 128 or not query.is_contiguous():
        raise ValueError("query must be a contiguous [query heads, 128] tensor")
    if key.ndim != 3 or key.shape != value.shape or key.shape[-1] != 128:
        raise ValueError("key and value must have shape [Hkv, S, 128]")
    if key.stride() != value.stride() or key.stride(-1) != 1:
        raise ValueError("key and value must share strides with a unit dim stride")
    if query.dtype != key.dtype or key.dtype != value.dtype or key.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("query, key and value must all be bf16 or all float32")
    return nat.KvCache(query.data_ptr(), key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1),
                       key.shape[1], query.shape[0], key.shape[0], nat.dtype_code(key.dtype), 0)


def csr_struct(csr) -> nat.PrefillCsr:
    if csr is None:
        return nat.PrefillCsr(None, None, 0)
    return nat.PrefillCsr(csr.member_offsets.data_ptr(), csr.member_positions.data_ptr(),
                          csr.member_positions.stride(0))


def delta_struct(deltas) -> nat.DeltaChunks:
    if deltas is None:
        return nat.DeltaChunks()
    return nat.DeltaChunks(*(t.data_ptr() for t in deltas.tensors()), deltas.position_capacity,
                           deltas.chunk_capacity_per_graph)


def state_struct(state, current_position: torch.Tensor) -> nat.GraphState:
    return nat.GraphState(
        state.centroids.data_ptr(), state.community_sizes.data_ptr(), state.community_counts.data_ptr(),
        state.community_weight.data_ptr(), state.total_weight.data_ptr(), state.token_communities.data_ptr(),
        state.retrieval_to_graph.data_ptr(), state.retrieval_to_kv.data_ptr(), current_position.data_ptr(),
        state.token_communities.shape[1], state.retrieval_head_count, state.graph_count,
        state.community_capacity, nat.dtype_code(state.centroids.dtype))


def config_struct(selection, *, group_size: int, sink_positions: torch.Tensor | None, softmax_scale: float,
                  lam: float, assignment: str) -> nat.DecodeConfig:
    mode = {"none": nat.CKV_ASSIGN_NONE, "delta_q": nat.CKV_ASSIGN_DELTA_Q,
            "nearest_centroid": nat.CKV_ASSIGN_NEAREST}[assignment]
    return nat.DecodeConfig(
        None if sink_positions is None or sink_positions.numel() == 0 else sink_positions.data_ptr(),
        group_size, selection.num_sink, selection.token_budget,
        nat.CKV_SELECT_BUDGET if selection.selection == "budget" else nat.CKV_SELECT_TOPK,
        selection.topk_communities, selection.selected_budget, selection.local_window,
        1 if selection.include_current else 0, mode, selection.score_coverage, float(softmax_scale), float(lam))


def workspace_struct(selection, attention, update) -> nat.DecodeWorkspace:
    def p(t):
        return None if t is None else t.data_ptr()

    return nat.DecodeWorkspace(
        p(selection.scores), p(selection.communities), p(selection.cumulative_ends),
        p(selection.descriptor_counts), p(selection.tile_descriptors), p(selection.selected_counts),
        p(selection.slot_positions), p(selection.exchange), p(selection.nearest),
        p(selection.block_counters),
        p(attention.partial_max) if attention else None, p(attention.partial_sum) if attention else None,
        p(attention.partial_acc) if attention else None, p(attention.slot_scores) if attention else None,
        p(attention.output) if attention else None, p(attention.lse) if attention else None,
        p(attention.topk_scores) if attention else None, p(attention.topk_positions) if attention else None,
        p(update.assigned_communities) if update else None, p(update.overflow) if update else None,
        selection.descriptor_capacity, selection.slot_capacity, selection.budget_tiles, selection.score_blocks)


@dataclass
class DecodeCall:
    """One packed argument set for the decode entry points."""

    kv: nat.KvCache
    state: nat.GraphState
    csr: nat.PrefillCsr
    deltas: nat.DeltaChunks
    config: nat.DecodeConfig
    workspace: nat.DecodeWorkspace
    device: torch.device
    keepalive: tuple = ()

    def _args(self, stream):
        return (ctypes.byref(self.kv), ctypes.byref(self.state), ctypes.byref(self.csr),
                ctypes.byref(self.deltas), ctypes.byref(self.config), ctypes.byref(self.workspace),
                ctypes.c_void_p(stream))

    def _stream(self, stream):
        return nat.stream_handle(self.device) if stream is None else stream

    def score_select(self, stream=None) -> None:
        nat.check(nat.lib().ckv_score_select(*self._args(self._stream(stream))))

    def attention(self, stream=None) -> None:
        nat.check(nat.lib().ckv_segmented_attention(*self._args(self._stream(stream))))

    def attention_partials(self, stream=None) -> None:
        nat.check(nat.lib().ckv_attention_partials(*self._args(self._stream(stream))))

    def layer_args(self) -> nat.LayerArgs:
        if getattr(self, "_layer_args", None) is None:
            self._layer_args = nat.LayerArgs(ctypes.pointer(self.kv), ctypes.pointer(self.state),
                                             ctypes.pointer(self.csr), ctypes.pointer(self.deltas),
                                             ctypes.pointer(self.config), ctypes.pointer(self.workspace))
        return self._layer_args

    def score_select_after(self, pending: "DecodeCall | None", stream=None) -> None:
        """Selection of this layer plus, in the same launch, the deferred
        online update of ``pending`` (another layer whose attention has run)."""
        nat.check(nat.lib().ckv_score_select_after_update(
            ctypes.byref(self.layer_args()), None if pending is None else ctypes.byref(pending.layer_args()),
            ctypes.c_void_p(self._stream(stream))))

    def decode_after(self, pending: "DecodeCall | None", stream=None) -> None:
        """Selection + attention of this layer (its update left pending) plus
        the deferred online update of ``pending`` in the same launches."""
        nat.check(nat.lib().ckv_decode_step_after_update(
            ctypes.byref(self.layer_args()), None if pending is None else ctypes.byref(pending.layer_args()),
            ctypes.c_void_p(self._stream(stream))))

    def select_attend_partials(self, stream=None) -> None:
        """The fused selection + attention-partials launch alone (profiling)."""
        nat.check(nat.lib().ckv_select_attend_partials(ctypes.byref(self.layer_args()),
                                                       ctypes.c_void_p(self._stream(stream))))

    def update(self, stream=None) -> None:
        nat.check(nat.lib().ckv_online_update(*self._args(self._stream(stream))))

    def decode(self, stream=None) -> None:
        nat.check(nat.lib().ckv_decode_layer(*self._args(self._stream(stream))))


class BatchDecode:
    """One decode step of several independent items (sequences of a ragged
    batch, or layers whose inputs are all ready) in four launches that cover
    all of them (``ckv_batch_decode``): selection, attention, split merge and
    online update.  The items' packed arguments are uploaded once to a device
    table (their tensors sit at fixed addresses); the step itself allocates
    nothing and does not synchronise."""

    def __init__(self, calls: "list[DecodeCall]") -> None:
        if not calls:
            raise ValueError("empty batch")
        self.calls = list(calls)
        self.device = calls[0].device
        self.items = (nat.LayerArgs * len(self.calls))(*[c.layer_args() for c in self.calls])
        size = int(nat.lib().ckv_batch_table_bytes(len(self.calls)))
        self.table = torch.empty(size, dtype=torch.uint8, device=self.device)
        nat.check(nat.lib().ckv_batch_prepare(self.items, len(self.calls), ctypes.c_void_p(self.table.data_ptr()),
                                              ctypes.c_void_p(nat.stream_handle(self.device))))

    def decode(self, stream=None) -> None:
        s = nat.stream_handle(self.device) if stream is None else stream
        nat.check(nat.lib().ckv_batch_decode(self.items, len(self.calls), ctypes.c_void_p(self.table.data_ptr()),
                                             ctypes.c_void_p(s)))

    def decode_after(self, pending: "BatchDecode | None", stream=None) -> None:
        """One step of this batch with its online update left pending, and
        the pending update of ``pending`` (another layer's batch whose step
        has run) in the same selection launch (``ckv_batch_decode_after_update``)."""
        s = nat.stream_handle(self.device) if stream is None else stream
        if pending is None:
            nat.check(nat.lib().ckv_batch_decode_after_update(
                self.items, len(self.calls), ctypes.c_void_p(self.table.data_ptr()), None, 0, None,
                ctypes.c_void_p(s)))
        else:
            nat.check(nat.lib().ckv_batch_decode_after_update(
                self.items, len(self.calls), ctypes.c_void_p(self.table.data_ptr()), pending.items,
                len(pending.calls), ctypes.c_void_p(pending.table.data_ptr()), ctypes.c_void_p(s)))

    def update(self, stream=None) -> None:
        """This batch's pending online update by itself (``ckv_batch_online_update``)."""
        s = nat.stream_handle(self.device) if stream is None else stream
        nat.check(nat.lib().ckv_batch_online_update(self.items, len(self.calls),
                                                    ctypes.c_void_p(self.table.data_ptr()), ctypes.c_void_p(s)))

    def attention_partials(self, stream=None) -> None:
        """The batched attention launch alone (profiling)."""
        s = nat.stream_handle(self.device) if stream is None else stream
        nat.check(nat.lib().ckv_batch_attention_partials(self.items, len(self.calls),
                                                         ctypes.c_void_p(self.table.data_ptr()), ctypes.c_void_p(s)))
