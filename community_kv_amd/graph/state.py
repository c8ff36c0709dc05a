"""Decode-time graph state layouts (reference: community_kv/graph/state.py:15-349).

The field names, dtypes and shapes are the reference's data contract: the HIP
kernels read and mutate exactly these tensors in place.  ``validate`` runs once
when a layer is prepared, never inside the decode step (the reference validated
on every step, with device-to-host syncs: graph/state.py:319-324).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


def _require_int32(name: str, value: torch.Tensor) -> None:
    if value.dtype != torch.int32:
        raise TypeError(f"{name} must use torch.int32")


@dataclass(slots=True)
class PrefillCSR:
    """Immutable community -> prefill-position index, newest position first."""

    member_offsets: torch.Tensor     # [graphs, community_capacity + 1]
    member_positions: torch.Tensor   # [graphs, members]
    community_counts: torch.Tensor   # [graphs]

    def validate(self) -> None:
        _require_int32("member_offsets", self.member_offsets)
        _require_int32("member_positions", self.member_positions)
        _require_int32("community_counts", self.community_counts)
        if self.member_offsets.ndim != 2 or self.member_positions.ndim != 2:
            raise ValueError("member offsets and positions must be rank two")
        if self.community_counts.shape != (self.member_offsets.shape[0],):
            raise ValueError("community_counts must have one entry per graph")
        if self.member_positions.shape[0] != self.member_offsets.shape[0]:
            raise ValueError("member_positions must have one row per graph")
        offsets = self.member_offsets.to(device="cpu", dtype=torch.int64)
        counts = self.community_counts.to(device="cpu", dtype=torch.int64)
        for graph in range(offsets.shape[0]):
            count = int(counts[graph])
            if count < 0 or count + 1 > offsets.shape[1]:
                raise ValueError("community count exceeds offset capacity")
            row = offsets[graph, : count + 1]
            if int(row[0]) != 0 or bool(torch.any(row[1:] < row[:-1])):
                raise ValueError("active CSR offsets must start at zero and be monotonic")
            if int(row[-1]) > self.member_positions.shape[1]:
                raise ValueError("CSR offsets exceed member-position capacity")

    @property
    def graph_count(self) -> int:
        return self.member_offsets.shape[0]

    @property
    def community_capacity(self) -> int:
        return self.member_offsets.shape[1] - 1

    def members(self, graph: int, community: int) -> torch.Tensor:
        if graph < 0 or graph >= self.graph_count:
            raise IndexError("graph is outside the CSR")
        count = int(self.community_counts[graph])
        if community < 0 or community >= count:
            raise IndexError("community is outside the active CSR")
        start = int(self.member_offsets[graph, community])
        end = int(self.member_offsets[graph, community + 1])
        return self.member_positions[graph, start:end]


_DELTA_FIELDS = (
    "positions", "chunk_start", "chunk_capacity", "chunk_size", "chunk_next", "chunk_previous",
    "community_head", "community_tail", "community_sizes", "next_free_chunk", "next_free_position",
)


@dataclass(slots=True)
class DecodeDeltaChunks:
    """Single-writer geometric chunk chains of decode-assigned positions.

    Chunk capacities of one community double (1, 2, 4, ...), so a community with
    n decode members has at most log2(n) + 1 chunks.
    """

    positions: torch.Tensor          # [graphs, 2 * max_decode_tokens]
    chunk_start: torch.Tensor        # [graphs, max_decode_tokens]
    chunk_capacity: torch.Tensor
    chunk_size: torch.Tensor
    chunk_next: torch.Tensor
    chunk_previous: torch.Tensor
    community_head: torch.Tensor     # [graphs, community_capacity]
    community_tail: torch.Tensor
    community_sizes: torch.Tensor
    next_free_chunk: torch.Tensor    # [graphs]
    next_free_position: torch.Tensor

    @classmethod
    def allocate(cls, *, graph_count: int, community_capacity: int, max_decode_tokens: int,
                 device: torch.device | str = "cpu") -> "DecodeDeltaChunks":
        if min(graph_count, community_capacity, max_decode_tokens) <= 0:
            raise ValueError("all capacities must be positive")
        chunks = (graph_count, max_decode_tokens)
        table = (graph_count, community_capacity)

        def full(shape, value):
            return torch.full(shape, value, dtype=torch.int32, device=device)

        return cls(
            positions=full((graph_count, 2 * max_decode_tokens), -1),
            chunk_start=full(chunks, -1),
            chunk_capacity=full(chunks, 0),
            chunk_size=full(chunks, 0),
            chunk_next=full(chunks, -1),
            chunk_previous=full(chunks, -1),
            community_head=full(table, -1),
            community_tail=full(table, -1),
            community_sizes=full(table, 0),
            next_free_chunk=full((graph_count,), 0),
            next_free_position=full((graph_count,), 0),
        )

    @property
    def graph_count(self) -> int:
        return self.positions.shape[0]

    @property
    def position_capacity(self) -> int:
        return self.positions.shape[1]

    @property
    def chunk_capacity_per_graph(self) -> int:
        return self.chunk_start.shape[1]

    @property
    def community_capacity(self) -> int:
        return self.community_head.shape[1]

    def tensors(self) -> tuple[torch.Tensor, ...]:
        return tuple(getattr(self, name) for name in _DELTA_FIELDS)

    def validate(self) -> None:
        for name in _DELTA_FIELDS:
            _require_int32(name, getattr(self, name))
            if not getattr(self, name).is_contiguous():
                raise ValueError(f"{name} must be contiguous")
        if self.positions.ndim != 2 or self.chunk_start.ndim != 2:
            raise ValueError("delta position and chunk pools must be rank two")
        graphs = self.positions.shape[0]
        if self.chunk_start.shape[0] != graphs or min(self.positions.shape[1:]) <= 0:
            raise ValueError("delta pool capacities must be positive")
        for value in (self.chunk_capacity, self.chunk_size, self.chunk_next, self.chunk_previous):
            if value.shape != self.chunk_start.shape:
                raise ValueError("chunk metadata shapes must match")
        if self.community_head.ndim != 2:
            raise ValueError("community chunk tables must be rank two")
        if self.community_head.shape != self.community_tail.shape:
            raise ValueError("community head and tail tables must match")
        if self.community_head.shape != self.community_sizes.shape:
            raise ValueError("community chunk tables and sizes must match")
        if self.community_head.shape[0] != graphs:
            raise ValueError("community chunk tables must match graph count")
        if self.next_free_chunk.shape != (graphs,):
            raise ValueError("next_free_chunk must have one entry per graph")
        if self.next_free_position.shape != (graphs,):
            raise ValueError("next_free_position must have one entry per graph")

    def append(self, graph: int, community: int, position: int) -> None:
        """Host-side append (one writer per graph); the device update kernel
        performs the same transition."""
        if graph < 0 or graph >= self.graph_count:
            raise IndexError("graph is outside the delta store")
        if community < 0 or community >= self.community_capacity:
            raise IndexError("community is outside the delta store")
        tail = int(self.community_tail[graph, community])
        size = int(self.chunk_size[graph, tail]) if tail >= 0 else 0
        cap = int(self.chunk_capacity[graph, tail]) if tail >= 0 else 0
        if tail < 0 or size == cap:
            chunk = int(self.next_free_chunk[graph])
            new_cap = 1 if tail < 0 else 2 * cap
            start = int(self.next_free_position[graph])
            if chunk >= self.chunk_capacity_per_graph:
                raise RuntimeError("decode-delta chunk capacity exhausted")
            if start + new_cap > self.position_capacity:
                raise RuntimeError("decode-delta position capacity exhausted")
            self.next_free_chunk[graph] = chunk + 1
            self.next_free_position[graph] = start + new_cap
            self.chunk_start[graph, chunk] = start
            self.chunk_capacity[graph, chunk] = new_cap
            self.chunk_previous[graph, chunk] = tail
            if tail < 0:
                self.community_head[graph, community] = chunk
            else:
                self.chunk_next[graph, tail] = chunk
            self.community_tail[graph, community] = chunk
            tail, size = chunk, 0
        self.positions[graph, int(self.chunk_start[graph, tail]) + size] = position
        self.chunk_size[graph, tail] = size + 1
        self.community_sizes[graph, community] += 1

    def members(self, graph: int, community: int) -> torch.Tensor:
        """Decode members of a community, oldest first."""
        size = int(self.community_sizes[graph, community])
        out = torch.empty((size,), dtype=torch.int32, device=self.positions.device)
        chunk = int(self.community_head[graph, community])
        cursor = 0
        while chunk >= 0 and cursor < size:
            n = int(self.chunk_size[graph, chunk])
            start = int(self.chunk_start[graph, chunk])
            out[cursor:cursor + n] = self.positions[graph, start:start + n]
            cursor += n
            chunk = int(self.chunk_next[graph, chunk])
        if cursor != size:
            raise RuntimeError("decode-delta chunk chain ended early")
        return out


@dataclass(slots=True)
class MutableGraphState:
    """Graph and centroid state mutated once per layer and decode token."""

    centroids: torch.Tensor           # [retrieval heads, C, 128] float8_e4m3fn (or float32)
    community_sizes: torch.Tensor     # [retrieval heads, C] int32
    community_counts: torch.Tensor    # [retrieval heads] int32
    community_weight: torch.Tensor    # [graphs, C] float32
    total_weight: torch.Tensor        # [graphs] float32
    token_communities: torch.Tensor   # [graphs, tokens] int32
    deltas: DecodeDeltaChunks
    retrieval_to_graph: torch.Tensor  # [retrieval heads] int32
    retrieval_to_kv: torch.Tensor     # [retrieval heads] int32

    @property
    def graph_count(self) -> int:
        return self.total_weight.shape[0]

    @property
    def retrieval_head_count(self) -> int:
        return self.centroids.shape[0]

    @property
    def community_capacity(self) -> int:
        return self.centroids.shape[1]

    @property
    def head_dim(self) -> int:
        return self.centroids.shape[2]

    def validate(self) -> None:
        if self.centroids.ndim != 3:
            raise ValueError("centroids must have shape [graphs, communities, dim]")
        if self.centroids.dtype not in (torch.float8_e4m3fn, torch.float32):
            raise TypeError("centroids must use FP8 E4M3 (or float32)")
        heads, capacity, _ = self.centroids.shape
        graphs = self.graph_count
        if self.community_sizes.shape != (heads, capacity):
            raise ValueError("community_sizes must match centroid rows")
        _require_int32("community_sizes", self.community_sizes)
        if self.community_counts.shape != (heads,):
            raise ValueError("community_counts must have one entry per retrieval head")
        _require_int32("community_counts", self.community_counts)
        if self.community_weight.shape != (graphs, capacity):
            raise ValueError("community_weight must have one row per graph")
        if self.community_weight.dtype != torch.float32:
            raise TypeError("community_weight must use float32")
        if self.total_weight.shape != (graphs,):
            raise ValueError("total_weight must have one entry per graph")
        if self.total_weight.dtype != torch.float32:
            raise TypeError("total_weight must use float32")
        if self.token_communities.ndim != 2 or self.token_communities.shape[0] != graphs:
            raise ValueError("token_communities must have one row per graph")
        _require_int32("token_communities", self.token_communities)
        self.deltas.validate()
        if self.deltas.graph_count != graphs:
            raise ValueError("delta pages must match graph count")
        if self.deltas.community_capacity != capacity:
            raise ValueError("delta pages must match community capacity")
        for name in ("retrieval_to_graph", "retrieval_to_kv"):
            mapping = getattr(self, name)
            _require_int32(name, mapping)
            if mapping.shape != (heads,):
                raise ValueError(f"{name} must have one entry per retrieval head")
        to_graph = self.retrieval_to_graph.cpu()
        if int(to_graph.min()) < 0 or int(to_graph.max()) >= graphs or int(self.retrieval_to_kv.min()) < 0:
            raise ValueError("retrieval mapping index is out of bounds")
        for r in range(heads):
            g = int(to_graph[r])
            if int(to_graph[g]) != g:
                raise ValueError("every graph must be owned by the retrieval head with its index")
        device = self.centroids.device
        tensors = (self.community_sizes, self.community_counts, self.community_weight, self.total_weight,
                   self.token_communities, self.retrieval_to_graph, self.retrieval_to_kv, *self.deltas.tensors())
        if any(t.device != device for t in tensors):
            raise ValueError("all mutable graph tensors must share one device")
        if any(not t.is_contiguous() for t in (self.centroids, *tensors)):
            raise ValueError("graph state tensors must be contiguous")


__all__ = ["DecodeDeltaChunks", "MutableGraphState", "PrefillCSR"]
