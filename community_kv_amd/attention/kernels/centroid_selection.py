"""Centroid scoring and exact community selection on the GPU.

Reference: attention/kernels/centroid_selection.py (workspace 191-327,
score_centroids 330-445, score_and_select 537-556) and
attention/kernels/_csrc/descriptor_selection.cu.  One HIP launch
(``ckv_score_select``) scores the query group against the centroid table and
runs the exact weighted selection; when the graph state is passed it also
materialises the KV position of every attended slot.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from community_kv_amd import _native as nat
from community_kv_amd.attention.kernels import _abi
from community_kv_amd.attention.kernels.packed_segments import ATTENTION_TILE, PackedSegments
from community_kv_amd.config import SELECTION_MODES

HEAD_DIM = 128
SCORE_BLOCK_N = nat.SCORE_BLOCK


def exchange_words(community_capacity: int) -> int:
    """uint64 words per retrieval head of the fused launch's exchange row:
    tagged scores, then tagged nearest-centroid minima (8 waves x 64 parts)
    and as many reserved words (ckv_exchange_words in csrc/ckv_device.h)."""
    return community_capacity + 2 * 64 * 8


@dataclass(slots=True)
class CentroidSelectionWorkspace:
    """Preallocated scoring/selection outputs and slot table."""

    scores: torch.Tensor            # [R, C] float16
    score_schedule: torch.Tensor | None
    communities: torch.Tensor       # [R, descriptor capacity] int32
    cumulative_ends: torch.Tensor   # [R, descriptor capacity] int32
    descriptor_counts: torch.Tensor  # [R] int32
    tile_descriptors: torch.Tensor  # [R, token_budget / 64] int32
    selected_counts: torch.Tensor   # [R] int32
    slot_positions: torch.Tensor    # [R, slot capacity] int32
    exchange: torch.Tensor          # [R, exchange_words(C)] uint64 (zeros): a fused launch's workgroups hand each
                                    # other centroid scores and nearest-centroid minima through it
    nearest: torch.Tensor           # [R] int32
    block_counters: torch.Tensor    # [4R] int32 arrival counters and epochs (zeros; kernel-maintained)
    token_budget: int
    num_sink: int
    score_coverage: int
    local_window: int = 0
    include_current: bool = True
    selection: str = "budget"
    topk_communities: int = 8
    max_selected: int = 0

    @classmethod
    def allocate(cls, *, kv_heads: int, community_capacity: int, token_budget: int, num_sink: int,
                 score_community_counts: Sequence[int] | None = None, score_headroom: int = 0,
                 device: torch.device | str, local_window: int = 0, include_current: bool = True,
                 selection: str = "budget", topk_communities: int = 8,
                 max_selected: int = 0) -> "CentroidSelectionWorkspace":
        if kv_heads <= 0 or community_capacity <= 0:
            raise ValueError("head and community capacities must be positive")
        if token_budget <= 0 or token_budget % ATTENTION_TILE:
            raise ValueError("token budget must be a positive multiple of 64")
        if num_sink < 0 or num_sink + 1 >= token_budget:
            raise ValueError("num_sink leaves no selected-token capacity")
        if num_sink > nat.MAX_SINKS or local_window > nat.MAX_WINDOW:
            raise ValueError(f"num_sink <= {nat.MAX_SINKS} and local_window <= {nat.MAX_WINDOW} are supported")
        if score_headroom < 0:
            raise ValueError("score_headroom must be nonnegative")
        if selection not in SELECTION_MODES:
            raise ValueError(f"selection must be one of {SELECTION_MODES}")
        if community_capacity > nat.MAX_COMMUNITIES:
            raise ValueError(f"community capacity above {nat.MAX_COMMUNITIES} is not supported")
        schedule = None
        coverage = community_capacity
        if score_community_counts is not None:
            if len(score_community_counts) != kv_heads:
                raise ValueError("score counts must contain one value per KV head")
            blocks, covered = [], []
            for head, count in enumerate(score_community_counts):
                if count <= 0 or count > community_capacity:
                    raise ValueError("score counts must fit the community capacity")
                cov = min(community_capacity, count + score_headroom)
                covered.append(cov)
                blocks.extend((head << 24) | b for b in range(-(-cov // SCORE_BLOCK_N)))
            schedule = torch.tensor(blocks, dtype=torch.int32, device=device)
            coverage = max(covered)
        inc = 1 if include_current else 0
        if selection == "budget":
            selected = token_budget - num_sink - inc
            dcap = min(selected, community_capacity)
        else:
            if max_selected <= 0 or topk_communities <= 0:
                raise ValueError("topk selection needs positive topk_communities and max_selected")
            selected = max_selected
            dcap = min(topk_communities, community_capacity)
        if dcap > nat.MAX_DESCRIPTORS:
            raise ValueError(f"descriptor capacity above {nat.MAX_DESCRIPTORS} is not supported")
        slots = num_sink + selected + local_window + inc
        slots = -(-slots // ATTENTION_TILE) * ATTENTION_TILE

        def i32(shape, value=0):
            return torch.full(shape, value, dtype=torch.int32, device=device)

        return cls(
            scores=torch.empty((kv_heads, community_capacity), dtype=torch.float16, device=device),
            score_schedule=schedule,
            communities=i32((kv_heads, dcap), -1),
            cumulative_ends=i32((kv_heads, dcap)),
            descriptor_counts=i32((kv_heads,)),
            tile_descriptors=i32((kv_heads, token_budget // ATTENTION_TILE)),
            selected_counts=i32((kv_heads,)),
            slot_positions=i32((kv_heads, slots), -1),
            exchange=torch.zeros((kv_heads, exchange_words(community_capacity)), dtype=torch.uint64,
                                 device=device),
            nearest=i32((kv_heads,), -1),
            block_counters=i32((4 * kv_heads,)),
            token_budget=token_budget,
            num_sink=num_sink,
            score_coverage=coverage,
            local_window=local_window,
            include_current=include_current,
            selection=selection,
            topk_communities=topk_communities,
            max_selected=max_selected,
        )

    @property
    def selected_budget(self) -> int:
        if self.selection == "budget":
            return self.token_budget - self.num_sink - (1 if self.include_current else 0)
        return self.max_selected

    @property
    def community_capacity(self) -> int:
        return self.scores.shape[1]

    @property
    def kv_heads(self) -> int:
        return self.scores.shape[0]

    @property
    def descriptor_capacity(self) -> int:
        return self.communities.shape[1]

    @property
    def slot_capacity(self) -> int:
        return self.slot_positions.shape[1]

    @property
    def budget_tiles(self) -> int:
        return self.tile_descriptors.shape[1]

    @property
    def score_blocks(self) -> int:
        return -(-self.score_coverage // SCORE_BLOCK_N)

    def packed_segments(self) -> PackedSegments:
        return PackedSegments(
            communities=self.communities,
            cumulative_ends=self.cumulative_ends,
            descriptor_counts=self.descriptor_counts,
            tile_descriptors=self.tile_descriptors,
            token_budget=self.token_budget,
            num_sink=self.num_sink,
            selected_counts=self.selected_counts,
            slot_positions=self.slot_positions,
        )


def _validate_scoring(query, centroids, community_sizes, community_counts, workspace) -> int:
    if query.ndim != 2 or query.shape[1] != HEAD_DIM or query.shape[0] % workspace.kv_heads:
        raise ValueError("query heads must divide into [KV head, group, 128]")
    group = query.shape[0] // workspace.kv_heads
    if not 1 <= group <= 16:
        raise ValueError("GQA group size must be in [1, 16]")
    if centroids.shape != (workspace.kv_heads, workspace.community_capacity, HEAD_DIM):
        raise ValueError("centroids have the wrong fixed capacity")
    if community_sizes.shape != centroids.shape[:2]:
        raise ValueError("community_sizes must match centroid rows")
    if community_counts.shape != (workspace.kv_heads,):
        raise ValueError("community_counts must have one entry per KV head")
    if query.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("query must use BF16 (or float32)")
    if centroids.dtype not in (torch.float8_e4m3fn, torch.float32):
        raise TypeError("centroids must use FP8 E4M3 (or float32)")
    if community_sizes.dtype != torch.int32 or community_counts.dtype != torch.int32:
        raise TypeError("community sizes and counts must use int32")
    return group


class _ScoringOnlyState:
    """Identity retrieval mapping for standalone scoring (no graph state)."""

    def __init__(self, centroids, community_sizes, community_counts):
        heads = centroids.shape[0]
        dev = centroids.device
        self.centroids = centroids
        self.community_sizes = community_sizes
        self.community_counts = community_counts
        self.community_weight = torch.zeros((1,), dtype=torch.float32, device=dev)
        self.total_weight = torch.zeros((heads,), dtype=torch.float32, device=dev)
        self.token_communities = torch.zeros((heads, 1), dtype=torch.int32, device=dev)
        self.retrieval_to_graph = torch.arange(heads, dtype=torch.int32, device=dev)
        self.retrieval_to_kv = self.retrieval_to_graph
        self.retrieval_head_count = heads
        self.graph_count = heads
        self.community_capacity = centroids.shape[1]
        self.current = torch.zeros((heads,), dtype=torch.int32, device=dev)


def score_and_select(*, query: torch.Tensor, centroids: torch.Tensor, community_sizes: torch.Tensor,
                     community_counts: torch.Tensor, workspace: CentroidSelectionWorkspace,
                     state=None, csr=None, current_position: torch.Tensor | None = None,
                     sink_positions: torch.Tensor | None = None, key: torch.Tensor | None = None,
                     value: torch.Tensor | None = None, assignment: str = "none") -> PackedSegments:
    """Scores and selects; with ``state``/``csr``/``current_position``/``key``
    also fills ``workspace.slot_positions`` for :func:`segmented_attention`."""
    group = _validate_scoring(query, centroids, community_sizes, community_counts, workspace)
    device = nat.require_device(query, centroids, community_sizes, community_counts, workspace.scores)
    if state is None:
        st = _ScoringOnlyState(centroids, community_sizes, community_counts)
        st_struct = _abi.state_struct(st, st.current)
        csr_s = _abi.csr_struct(None)
        dl_s = _abi.delta_struct(None)
        kv_key = torch.zeros((1, 1, HEAD_DIM), dtype=query.dtype, device=device)
        kv = _abi.kv_struct(query, kv_key, kv_key)
        keep = (st, kv_key)
    else:
        if csr is None or current_position is None or key is None:
            raise ValueError("slot materialisation needs csr, current_position and key")
        st_struct = _abi.state_struct(state, current_position)
        csr_s = _abi.csr_struct(csr)
        dl_s = _abi.delta_struct(state.deltas)
        kv = _abi.kv_struct(query, key, key if value is None else value)
        keep = ()
    cfg = _abi.config_struct(workspace, group_size=group, sink_positions=sink_positions, softmax_scale=1.0,
                             lam=0.0, assignment=assignment)
    ws = _abi.workspace_struct(workspace, None, None)
    call = _abi.DecodeCall(kv, st_struct, csr_s, dl_s, cfg, ws, device, keep)
    call.score_select()
    return workspace.packed_segments()


def score_centroids(*, query: torch.Tensor, centroids: torch.Tensor, community_sizes: torch.Tensor,
                    community_counts: torch.Tensor, workspace: CentroidSelectionWorkspace) -> torch.Tensor:
    """fp16 scores [R, C]: max over the query group of q . centroid; -inf for
    inactive or empty communities (centroid_selection.py:32-108)."""
    score_and_select(query=query, centroids=centroids, community_sizes=community_sizes,
                     community_counts=community_counts, workspace=workspace)
    return workspace.scores


__all__ = ["CentroidSelectionWorkspace", "score_and_select", "score_centroids"]
