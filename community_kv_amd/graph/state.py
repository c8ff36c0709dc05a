"""Decode-time graph state (reference data contract: community_kv/graph/state.py:15-349).

The field names, dtypes and shapes are the reference's: the partitioner
produces these tensors and the HIP kernels read and mutate them in place.
Each class states its layout once, as a table of (field, dtypes, dimension
names); ``validate`` checks every field against the table, binding each
dimension name to the first extent it meets, so two fields that share a name
must agree.  Validation runs once when a layer is prepared, never inside the
decode step.
"""

from __future__ import annotations

from dataclasses import dataclass, fields

import torch

I32 = (torch.int32,)
F32 = (torch.float32,)


def _check_layout(obj, layout, dims: dict[str, int] | None = None) -> dict[str, int]:
    """Checks each (field, dtypes, dimension names) of ``layout`` on ``obj``;
    returns the bound extents.  A None entry in the names skips that dimension."""
    dims = {} if dims is None else dims
    kind = type(obj).__name__
    for name, dtypes, names in layout:
        t = getattr(obj, name)
        if t.dtype not in dtypes:
            raise TypeError(f"{kind}.{name} has dtype {t.dtype}; expected {' or '.join(map(str, dtypes))}")
        if t.ndim != len(names):
            raise ValueError(f"{kind}.{name} has rank {t.ndim}; expected {len(names)} ({', '.join(map(str, names))})")
        for axis, dim in enumerate(names):
            if dim is None:
                continue
            extent = int(t.shape[axis])
            if dims.setdefault(dim, extent) != extent:
                raise ValueError(f"{kind}.{name} dimension {axis} is {extent}, but {dim} is {dims[dim]} elsewhere")
    return dims


@dataclass(slots=True)
class PrefillCSR:
    """Immutable community -> prefill positions index (each row newest first)."""

    member_offsets: torch.Tensor     # [graphs, community_capacity + 1]
    member_positions: torch.Tensor   # [graphs, members]
    community_counts: torch.Tensor   # [graphs]

    LAYOUT = (("member_offsets", I32, ("graphs", "offsets")),
              ("member_positions", I32, ("graphs", "members")),
              ("community_counts", I32, ("graphs",)))

    def validate(self) -> None:
        dims = _check_layout(self, self.LAYOUT)
        offsets = self.member_offsets.to("cpu", torch.int64)
        counts = self.community_counts.to("cpu", torch.int64).tolist()
        for graph, count in enumerate(counts):
            if not 0 <= count < dims["offsets"]:
                raise ValueError(f"graph {graph}: {count} active communities do not fit {dims['offsets'] - 1} offsets")
            active = offsets[graph, : count + 1]
            steps = active[1:] - active[:-1]
            if int(active[0]) != 0 or bool((steps < 0).any()):
                raise ValueError(f"graph {graph}: active CSR offsets must start at 0 and never decrease")
            if int(active[-1]) > dims["members"]:
                raise ValueError(f"graph {graph}: CSR offsets reach {int(active[-1])} of {dims['members']} members")

    @property
    def graph_count(self) -> int:
        return self.member_offsets.shape[0]

    @property
    def community_capacity(self) -> int:
        return self.member_offsets.shape[1] - 1

    def members(self, graph: int, community: int) -> torch.Tensor:
        """Prefill members of one active community, newest first."""
        if not 0 <= graph < self.graph_count:
            raise IndexError("graph is outside the CSR")
        if not 0 <= community < int(self.community_counts[graph]):
            raise IndexError("community is outside the active CSR")
        lo, hi = (int(x) for x in self.member_offsets[graph, community:community + 2])
        return self.member_positions[graph, lo:hi]


@dataclass(slots=True)
class DecodeDeltaChunks:
    """Per-graph pools of decode-assigned positions, chained per community.

    A community's chunks double in capacity (1, 2, 4, ...), so n decode members
    take at most log2(n) + 1 chunks; every append touches only its own
    community's tail chunk (one writer per graph: the graph's owner head).
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

    LAYOUT = (("positions", I32, ("graphs", "position_pool")),
              *((name, I32, ("graphs", "chunks")) for name in
                ("chunk_start", "chunk_capacity", "chunk_size", "chunk_next", "chunk_previous")),
              *((name, I32, ("graphs", "communities")) for name in
                ("community_head", "community_tail", "community_sizes")),
              ("next_free_chunk", I32, ("graphs",)),
              ("next_free_position", I32, ("graphs",)))

    @classmethod
    def allocate(cls, *, graph_count: int, community_capacity: int, max_decode_tokens: int,
                 device: torch.device | str = "cpu") -> "DecodeDeltaChunks":
        if min(graph_count, community_capacity, max_decode_tokens) <= 0:
            raise ValueError("graph count, community capacity and decode tokens must all be positive")
        extent = {"position_pool": 2 * max_decode_tokens, "chunks": max_decode_tokens,
                  "communities": community_capacity}
        unset = {"positions": -1, "chunk_start": -1, "chunk_next": -1, "chunk_previous": -1,
                 "community_head": -1, "community_tail": -1}
        made = {}
        for name, _, names in cls.LAYOUT:
            shape = tuple(graph_count if d == "graphs" else extent[d] for d in names)
            made[name] = torch.full(shape, unset.get(name, 0), dtype=torch.int32, device=device)
        return cls(**made)

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
        """The fields in declaration order (the C ABI's order)."""
        return tuple(getattr(self, f.name) for f in fields(self))

    def validate(self) -> None:
        dims = _check_layout(self, self.LAYOUT)
        if min(dims["position_pool"], dims["chunks"]) <= 0:
            raise ValueError("the delta position and chunk pools must not be empty")
        loose = [f.name for f in fields(self) if not getattr(self, f.name).is_contiguous()]
        if loose:
            raise ValueError(f"delta fields must be contiguous: {loose}")

    def _open_chunk(self, graph: int, community: int, after: int, capacity: int) -> int:
        """Takes the graph's next free chunk (and `capacity` pool slots) and
        links it behind chunk `after` (-1: the community's first)."""
        chunk = int(self.next_free_chunk[graph])
        start = int(self.next_free_position[graph])
        if chunk >= self.chunk_capacity_per_graph:
            raise RuntimeError(f"graph {graph}: all {self.chunk_capacity_per_graph} decode-delta chunks are in use")
        if start + capacity > self.position_capacity:
            raise RuntimeError(f"graph {graph}: the decode-delta position pool is full")
        self.next_free_chunk[graph] = chunk + 1
        self.next_free_position[graph] = start + capacity
        self.chunk_start[graph, chunk] = start
        self.chunk_capacity[graph, chunk] = capacity
        self.chunk_previous[graph, chunk] = after
        (self.community_head if after < 0 else self.chunk_next)[graph, community if after < 0 else after] = chunk
        self.community_tail[graph, community] = chunk
        return chunk

    def append(self, graph: int, community: int, position: int) -> None:
        """Host-side append; the device update kernel makes the same transition."""
        if not 0 <= graph < self.graph_count:
            raise IndexError(f"graph {graph} is outside the delta store")
        if not 0 <= community < self.community_capacity:
            raise IndexError(f"community {community} is outside the delta store")
        tail = int(self.community_tail[graph, community])
        if tail < 0:
            tail = self._open_chunk(graph, community, -1, 1)
        elif int(self.chunk_size[graph, tail]) == int(self.chunk_capacity[graph, tail]):
            tail = self._open_chunk(graph, community, tail, 2 * int(self.chunk_capacity[graph, tail]))
        fill = int(self.chunk_size[graph, tail])
        self.positions[graph, int(self.chunk_start[graph, tail]) + fill] = position
        self.chunk_size[graph, tail] = fill + 1
        self.community_sizes[graph, community] += 1

    def members(self, graph: int, community: int) -> torch.Tensor:
        """Decode members of a community in append order (oldest first)."""
        parts = []
        chunk = int(self.community_head[graph, community])
        while chunk >= 0:
            start = int(self.chunk_start[graph, chunk])
            parts.append(self.positions[graph, start:start + int(self.chunk_size[graph, chunk])])
            chunk = int(self.chunk_next[graph, chunk])
        out = torch.cat(parts) if parts else self.positions.new_empty((0,))
        if out.numel() != int(self.community_sizes[graph, community]):
            raise RuntimeError(f"graph {graph}, community {community}: the chunk chain holds {out.numel()} of "
                               f"{int(self.community_sizes[graph, community])} members")
        return out


@dataclass(slots=True)
class MutableGraphState:
    """Graph and centroid state that every decode token updates."""

    centroids: torch.Tensor           # [retrieval heads, C, 128] float8_e4m3fn (or float32)
    community_sizes: torch.Tensor     # [retrieval heads, C] int32
    community_counts: torch.Tensor    # [retrieval heads] int32
    community_weight: torch.Tensor    # [graphs, C] float32
    total_weight: torch.Tensor        # [graphs] float32
    token_communities: torch.Tensor   # [graphs, tokens] int32
    deltas: DecodeDeltaChunks
    retrieval_to_graph: torch.Tensor  # [retrieval heads] int32
    retrieval_to_kv: torch.Tensor     # [retrieval heads] int32

    LAYOUT = (("centroids", (torch.float8_e4m3fn, torch.float32), ("heads", "communities", None)),
              ("community_sizes", I32, ("heads", "communities")),
              ("community_counts", I32, ("heads",)),
              ("community_weight", F32, ("graphs", "communities")),
              ("total_weight", F32, ("graphs",)),
              ("token_communities", I32, ("graphs", None)),
              ("retrieval_to_graph", I32, ("heads",)),
              ("retrieval_to_kv", I32, ("heads",)))

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

    def _tensors(self) -> list[torch.Tensor]:
        return [getattr(self, name) for name, _, _ in self.LAYOUT] + list(self.deltas.tensors())

    def validate(self) -> None:
        dims = _check_layout(self, self.LAYOUT)
        self.deltas.validate()
        # the delta store is indexed by graph and community like the tables above
        _check_layout(self.deltas, (("community_sizes", I32, ("graphs", "communities")),), dims)
        to_graph = self.retrieval_to_graph.cpu().tolist()
        if any(not 0 <= g < dims["graphs"] for g in to_graph) or int(self.retrieval_to_kv.min()) < 0:
            raise ValueError(f"retrieval head mappings point outside the {dims['graphs']} graphs / KV heads")
        owners = [g for g in to_graph if to_graph[g] != g]
        if owners:
            raise ValueError(f"graph {owners[0]} is not owned by the retrieval head of the same index")
        tensors = self._tensors()
        if len({t.device for t in tensors}) != 1:
            raise ValueError("the graph state spans several devices")
        if not all(t.is_contiguous() for t in tensors):
            raise ValueError("graph state tensors must be contiguous")


__all__ = ["DecodeDeltaChunks", "MutableGraphState", "PrefillCSR"]
