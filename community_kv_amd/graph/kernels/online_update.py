"""Workspace of the fused online update (reference: graph/kernels/online_update.py:10-35)."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from community_kv_amd.config import ASSIGNMENT_MODES


@dataclass(slots=True)
class OnlineUpdateWorkspace:
    assigned_communities: torch.Tensor  # [graphs] int32, -1 on community overflow
    overflow: torch.Tensor              # [graphs] int32 bit flags
    assignment: str = "delta_q"

    @classmethod
    def allocate(cls, *, graph_count: int, device: torch.device | str,
                 assignment: str = "delta_q") -> "OnlineUpdateWorkspace":
        if graph_count <= 0:
            raise ValueError("graph_count must be positive")
        if assignment not in ASSIGNMENT_MODES + ("none",):
            raise ValueError(f"assignment must be one of {ASSIGNMENT_MODES + ('none',)}")
        return cls(
            assigned_communities=torch.full((graph_count,), -1, dtype=torch.int32, device=device),
            overflow=torch.zeros((graph_count,), dtype=torch.int32, device=device),
            assignment=assignment,
        )


__all__ = ["OnlineUpdateWorkspace"]
