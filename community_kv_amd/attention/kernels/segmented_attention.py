"""Segmented GQA decode attention + fused online update on the GPU.

Reference: attention/kernels/segmented_attention.py (workspace 953-1013,
triton_segmented_attention 1016-1273).  The HIP entry point
``ckv_segmented_attention`` runs the split partials over the slot table that
``score_and_select`` materialised, the split merge, and (unless the workspace's
assignment is ``"none"``) the online update of the graph state.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from community_kv_amd import _native as nat
from community_kv_amd.attention.kernels import _abi
from community_kv_amd.attention.kernels.packed_segments import ATTENTION_TILE, PackedSegments

HEAD_DIM = 128
KAPPA = 8
BLOCK_N = ATTENTION_TILE


@dataclass(slots=True)
class SegmentedAttentionWorkspace:
    group_size: int
    partial_max: torch.Tensor          # [Hq, tiles] float32
    partial_sum: torch.Tensor          # [Hq, tiles] float32
    partial_acc: torch.Tensor          # [Hq, tiles, 128] float32
    partial_topk_packed: torch.Tensor  # [R, tiles, 8] uint64: the reference's shape, as a zero-stride view (no
                                       # memory): the kernels take the top-8 from slot_scores instead
    slot_scores: torch.Tensor          # [R, slot capacity] float32: first query's score per slot (top-8 candidates)
    output: torch.Tensor               # [Hq, 128]
    lse: torch.Tensor                  # [Hq] float32
    topk_scores: torch.Tensor          # [R, 8] float32
    topk_positions: torch.Tensor       # [R, 8] int32

    @classmethod
    def allocate(cls, *, kv_heads: int, group_size: int = 4, token_budget: int, dtype: torch.dtype,
                 device: torch.device | str, slot_capacity: int | None = None) -> "SegmentedAttentionWorkspace":
        if kv_heads <= 0:
            raise ValueError("kv_heads must be positive")
        if not 1 <= group_size <= 16:
            raise ValueError("group_size must be in [1, 16]")
        if token_budget <= 0 or token_budget % BLOCK_N:
            raise ValueError("token_budget must be a positive multiple of 64")
        if dtype not in (torch.bfloat16, torch.float32):
            raise TypeError("Q/K/V must use BF16 (or float32)")
        slots = token_budget if slot_capacity is None else slot_capacity
        if slots % BLOCK_N:
            raise ValueError("slot capacity must be a multiple of 64")
        heads = kv_heads * group_size
        tiles = slots // BLOCK_N
        return cls(
            group_size=group_size,
            partial_max=torch.empty((heads, tiles), dtype=torch.float32, device=device),
            partial_sum=torch.empty((heads, tiles), dtype=torch.float32, device=device),
            partial_acc=torch.empty((heads, tiles, HEAD_DIM), dtype=torch.float32, device=device),
            partial_topk_packed=torch.zeros((), dtype=torch.uint64, device=device).expand(kv_heads, tiles, KAPPA),
            slot_scores=torch.empty((kv_heads, slots), dtype=torch.float32, device=device),
            output=torch.empty((heads, HEAD_DIM), dtype=dtype, device=device),
            lse=torch.empty((heads,), dtype=torch.float32, device=device),
            topk_scores=torch.empty((kv_heads, KAPPA), dtype=torch.float32, device=device),
            topk_positions=torch.empty((kv_heads, KAPPA), dtype=torch.int32, device=device),
        )


def segmented_attention(*, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, csr, deltas,
                        segments: PackedSegments, sink_positions: torch.Tensor, current_position: torch.Tensor,
                        softmax_scale: float, workspace: SegmentedAttentionWorkspace, update_state,
                        update_workspace, update_lam: float, selection=None):
    """Attention over the slots chosen by the preceding ``score_and_select``
    (which must have been given the same graph state), then the fused update.
    Returns (output, lse, topk_scores, topk_positions)."""
    retrieval_heads = workspace.topk_scores.shape[0]
    if query.shape != (retrieval_heads * workspace.group_size, HEAD_DIM):
        raise ValueError(f"query must have {workspace.group_size} [128] heads per retrieval head")
    if key.ndim != 3 or value.shape != key.shape or key.shape[-1] != HEAD_DIM:
        raise ValueError("key and value must have shape [Hkv, S, 128]")
    if query.dtype != key.dtype:
        raise TypeError("query, key, and value must share a dtype")
    if segments.token_budget % BLOCK_N:
        raise ValueError("token budget must be a multiple of 64")
    if selection is None or segments.slot_positions is None:
        raise ValueError("segmented_attention needs the selection workspace that produced the slot table")
    if update_state.deltas is not deltas:
        raise ValueError("fused update must mutate the attention delta store")
    if not 0.0 <= update_lam <= 1.0:
        raise ValueError("update_lam must be in [0, 1]")
    device = nat.require_device(query, key, value, current_position)
    call = _abi.DecodeCall(
        _abi.kv_struct(query, key, value), _abi.state_struct(update_state, current_position), _abi.csr_struct(csr),
        _abi.delta_struct(deltas),
        _abi.config_struct(selection, group_size=workspace.group_size, sink_positions=sink_positions,
                           softmax_scale=softmax_scale, lam=update_lam, assignment=update_workspace.assignment),
        _abi.workspace_struct(selection, workspace, update_workspace), device)
    call.attention()
    call.update()
    return workspace.output, workspace.lse, workspace.topk_scores, workspace.topk_positions


# Reference names (attention/kernels/segmented_attention.py:953, 1016).
TritonSegmentedAttentionWorkspace = SegmentedAttentionWorkspace
triton_segmented_attention = segmented_attention

__all__ = [
    "SegmentedAttentionWorkspace",
    "TritonSegmentedAttentionWorkspace",
    "segmented_attention",
    "triton_segmented_attention",
]
