"""Selected-community descriptors (reference: attention/kernels/packed_segments.py:9-21)."""

from __future__ import annotations

from dataclasses import dataclass

import torch

ATTENTION_TILE = 64


@dataclass(frozen=True, slots=True)
class PackedSegments:
    """Device tensors describing one step's selection.

    ``communities``/``cumulative_ends`` list the selected communities in the
    reference's descriptor order with the running member count; ``tile_descriptors``
    holds, per 64-slot tile, the first descriptor the tile touches.
    ``slot_positions`` (this build) is the KV position of every attended slot.
    """

    communities: torch.Tensor
    cumulative_ends: torch.Tensor
    descriptor_counts: torch.Tensor
    tile_descriptors: torch.Tensor
    token_budget: int
    num_sink: int
    selected_counts: torch.Tensor | None = None
    slot_positions: torch.Tensor | None = None


__all__ = ["ATTENTION_TILE", "PackedSegments"]
