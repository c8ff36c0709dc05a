"""Shared test helpers: move oracle fixtures to the device and compare states."""

from __future__ import annotations

import numpy as np
import torch

from community_kv_amd.attention.decode import DecodeLayerWorkspace
from community_kv_amd.graph.state import DecodeDeltaChunks, MutableGraphState, PrefillCSR
from oracle import ckv_oracle as co
from oracle import numerics as nm


def torch_values(x: np.ndarray, dtype: str, device) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(device=device, dtype=torch.bfloat16 if dtype == "bf16" else torch.float32)


def to_device(fx, device):
    """Oracle LayerFixture -> (state, csr, current_position, query, key, value) on device."""
    st = fx.state
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(device)
    if st.fp8:
        cent = torch.from_numpy(np.ascontiguousarray(st.centroids)).view(torch.float8_e4m3fn).to(device)
    else:
        cent = torch.from_numpy(np.ascontiguousarray(st.centroids, dtype=np.float32)).to(device)
    d = st.deltas
    deltas = DecodeDeltaChunks(*(i32(getattr(d, f)) for f in (
        "positions", "chunk_start", "chunk_capacity", "chunk_size", "chunk_next", "chunk_previous",
        "community_head", "community_tail", "community_sizes", "next_free_chunk", "next_free_position")))
    state = MutableGraphState(
        centroids=cent, community_sizes=i32(st.community_sizes), community_counts=i32(st.community_counts),
        community_weight=torch.from_numpy(st.community_weight.copy()).to(device),
        total_weight=torch.from_numpy(st.total_weight.copy()).to(device),
        token_communities=i32(st.token_communities), deltas=deltas, retrieval_to_graph=i32(st.to_graph),
        retrieval_to_kv=i32(st.to_kv))
    counts = np.zeros(len(st.total_weight), np.int32)
    for r in range(st.retrieval_heads):
        counts[st.to_graph[r]] = st.community_counts[r]
    csr = PrefillCSR(i32(st.member_offsets), i32(st.member_positions), i32(counts))
    current = i32(st.current_position)
    q = torch_values(fx.query, fx.dtype, device)
    k = torch_values(fx.keys, fx.dtype, device)
    v = torch_values(fx.values, fx.dtype, device)
    return state, csr, current, q, k, v


def workspace_for(fx, params: co.StepParams, device, *, headroom=None):
    st = fx.state
    cap = st.community_capacity
    counts = [int(c) for c in st.community_counts]
    headroom = st.deltas.chunk_start.shape[1] if headroom is None else headroom
    return DecodeLayerWorkspace.allocate(
        retrieval_head_count=st.retrieval_heads, graph_count=len(st.total_weight), group_size=params.group_size,
        community_capacity=cap, token_budget=params.token_budget, num_sink=params.num_sink,
        dtype=torch.bfloat16 if fx.dtype == "bf16" else torch.float32, device=device,
        score_community_counts=counts, score_headroom=headroom, local_window=params.local_window,
        include_current=params.include_current, selection=params.mode, topk_communities=params.topk_communities,
        max_selected=params.max_selected, assignment=params.assignment)


def state_to_numpy(state: MutableGraphState, current: torch.Tensor, fp8: bool) -> dict:
    out = {
        "centroids": (state.centroids.view(torch.uint8) if fp8 else state.centroids).cpu().numpy(),
        "community_sizes": state.community_sizes.cpu().numpy(),
        "community_counts": state.community_counts.cpu().numpy(),
        "community_weight": state.community_weight.cpu().numpy(),
        "total_weight": state.total_weight.cpu().numpy(),
        "token_communities": state.token_communities.cpu().numpy(),
        "current_position": current.cpu().numpy(),
    }
    for f in ("positions", "chunk_start", "chunk_capacity", "chunk_size", "chunk_next", "chunk_previous",
              "community_head", "community_tail", "community_sizes", "next_free_chunk", "next_free_position"):
        out["delta_" + f] = getattr(state.deltas, f).cpu().numpy()
    return out


def oracle_state_dict(st: co.LayerState) -> dict:
    out = {
        "centroids": st.centroids,
        "community_sizes": st.community_sizes,
        "community_counts": st.community_counts,
        "community_weight": st.community_weight,
        "total_weight": st.total_weight,
        "token_communities": st.token_communities,
        "current_position": st.current_position,
    }
    for f in ("positions", "chunk_start", "chunk_capacity", "chunk_size", "chunk_next", "chunk_previous",
              "community_head", "community_tail", "community_sizes", "next_free_chunk", "next_free_position"):
        out["delta_" + f] = getattr(st.deltas, f)
    return out


def assert_states_equal(device_state: dict, oracle_state: dict) -> None:
    for name, ref in oracle_state.items():
        got = device_state[name]
        if ref.dtype == np.float32:
            ok = np.array_equal(got.view(np.uint32), np.asarray(ref, np.float32).view(np.uint32))
        else:
            ok = np.array_equal(got, ref)
        if not ok:
            diff = np.argwhere(np.asarray(got) != np.asarray(ref))
            raise AssertionError(f"state field {name} differs at {diff[:5].tolist()}")


def descriptor_lists(ws_sel, r):
    n = int(ws_sel.descriptor_counts[r])
    return (ws_sel.communities[r, :n].cpu().tolist(), ws_sel.cumulative_ends[r, :n].cpu().tolist())


def check_topk(gpu_pos, gpu_scores, oracle_scores0, positions, num_sink, tol=1e-4):
    """GPU top-8 positions must be a valid top-8 of the oracle's float64 scores,
    allowing swaps only between entries whose scores are within ``tol``."""
    pos = np.asarray(positions)
    cand = {int(pos[i]): float(oracle_scores0[i]) for i in range(len(pos)) if i >= num_sink and pos[i] >= 0}
    ranked = sorted(cand.items(), key=lambda kv: (-kv[1], kv[0]))
    k = min(8, len(ranked))
    kth = ranked[k - 1][1]
    got = [int(p) for p in gpu_pos[:k]]
    assert len(set(got)) == k, f"duplicate top-k positions {got}"
    for p, s in zip(got, gpu_scores[:k]):
        assert p in cand, f"top-k position {p} is not an attended candidate"
        assert cand[p] >= kth - tol, f"position {p} score {cand[p]} below the 8th best {kth}"
        assert abs(cand[p] - float(s)) <= tol * max(1.0, abs(cand[p])), "top-k score mismatch"
    for p, s in ranked[:k]:
        if p not in got:
            assert s <= kth + tol, f"missed candidate {p} with score {s} (8th best {kth})"
