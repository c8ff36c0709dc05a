"""Native batched Leiden (ckv_batched_leiden, ckv_aggregate_coo,
ckv_densify_*) against the oracle's restatement of the reference
(oracle/leiden.py).  Dyadic edge weights make every float sum exact, so labels
must match bit for bit; with arbitrary float weights the sums are formed in
another order and the labels are still expected to match (a flip needs two
gains within an ulp)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from community_kv_amd.graph.leiden import algorithm
from oracle import leiden as L
from tests import _leiden_graphs as lg

pytestmark = pytest.mark.gpu


def _dev(device, *arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in arrays]


def _native_level(device, src, dst, w, G, S, **kw):
    s, d, x = _dev(device, src, dst, w)
    mod = algorithm._load_module()
    labels, q = mod.batched_leiden(s, d, x, G, S, 6, kw.get("resolution", 1.0), kw.get("theta", 0.01),
                                   kw.get("max_inner_iter", 16), kw.get("seed", 0), kw.get("use_boltzmann", False))
    torch.cuda.synchronize()
    return labels.cpu().numpy(), q.cpu().numpy()


LEVEL_CASES = [
    # seed, graphs, seq_len, communities, kwargs for planted(), kwargs for Leiden
    (1, 3, 500, 8, dict(), dict()),
    (2, 2, 800, 12, dict(self_loops=6, isolated=7, duplicates=20), dict(max_inner_iter=4)),
    (3, 4, 300, 5, dict(edges_per_vertex=10.0), dict(resolution=0.5, seed=7)),
    (4, 1, 2000, 30, dict(p_in=0.6), dict(resolution=2.0, max_inner_iter=1)),
    (5, 2, 600, 10, dict(dyadic=False), dict()),
    (6, 3, 400, 6, dict(dyadic=False, self_loops=3), dict(resolution=1.5, seed=3)),
]


@pytest.mark.parametrize("seed,G,S,k,gkw,lkw", LEVEL_CASES)
def test_batched_leiden_level_matches_oracle(device, seed, G, S, k, gkw, lkw):
    print(f"leiden level seed={seed} G={G} S={S} {gkw} {lkw}", flush=True)
    src, dst, w = lg.planted(seed, G, S, k, **gkw)
    got, q = _native_level(device, src, dst, w, G, S, **lkw)
    ref, q_ref = L.batched_leiden(src, dst, w, graphs=G, seq_len=S, **lkw)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_allclose(q, q_ref, rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize("leaves", [3000, 1500, 1100, 300, 100])
def test_hub_vertex_over_table_capacity(device, leaves):
    """Degree 3000, 1500 and 1100 (workgroup kernel: the row is walked 1024
    entries at a time and the first 1024 communities along it are kept), 300
    (hub kernel, hashed table) and 100 (small-row kernel).  The workgroup
    table never overflows; if it did, the call would mark its modularity NaN
    (checked finite here) and run_leiden would raise."""
    src, dst, w, S = lg.hub(4, leaves, 40)
    print(f"leiden hub S={S} edges={src.size}", flush=True)
    got, q = _native_level(device, src, dst, w, 1, S)
    ref, _ = L.batched_leiden(src, dst, w, graphs=1, seq_len=S)
    np.testing.assert_array_equal(got, ref)
    assert np.isfinite(q).all()


def test_boltzmann_refinement_close_to_oracle(device):
    """Gumbel noise goes through logf: the device and numpy logarithms may
    differ in the last ulp, which can move a near-tied sample."""
    src, dst, w = lg.planted(8, 2, 700, 9)
    print("leiden boltzmann", flush=True)
    got, q = _native_level(device, src, dst, w, 2, 700, use_boltzmann=True, theta=0.05, seed=5)
    ref, q_ref = L.batched_leiden(src, dst, w, graphs=2, seq_len=700, use_boltzmann=True, theta=0.05, seed=5)
    assert (got == ref).mean() > 0.98
    np.testing.assert_allclose(q, q_ref, atol=5e-3)


def test_no_edges_marks_every_vertex_isolated(device):
    e = np.zeros(0, np.int32)
    got, q = _native_level(device, e, e, np.zeros(0, np.float32), 2, 5)
    assert (got == -1).all() and (q == 0).all()


def test_aggregate_coo_matches_oracle(device):
    src, dst, w = lg.planted(12, 3, 400, 7, self_loops=5)
    lab, _ = L.batched_leiden(src, dst, w, graphs=3, seq_len=400)
    lab = np.where(lab < 0, np.arange(1200), lab).astype(np.int32)
    dense, width = L.densify_per_graph(lab, 3, 400)
    print(f"aggregate width={width}", flush=True)
    s, d, x, dl = _dev(device, src, dst, w, dense)
    out = algorithm._load_module().aggregate_coo(s, d, x, dl, 3 * width)
    ref = L.aggregate_coo(src, dst, w, dense, 3 * width)
    for a, b in zip(out[:2], ref[:2]):
        np.testing.assert_array_equal(a.cpu().numpy(), b)
    np.testing.assert_array_equal(out[2].cpu().numpy(), ref[2])  # dyadic: exact sums


def test_densify_matches_oracle(device):
    rng = np.random.default_rng(3)
    G, S = 4, 777
    lab = (rng.integers(0, 50, (G, S)) * 7 % S + np.arange(G)[:, None] * S).astype(np.int32).ravel()
    lab[rng.random(lab.size) < 0.05] = -1
    print("densify", flush=True)
    dense, width = algorithm._densify_per_graph(torch.from_numpy(lab).to(device), G, S)
    own = np.where(lab < 0, np.arange(G * S), lab)
    ref, ref_w = L.densify_per_graph(own, G, S)
    assert width == ref_w
    np.testing.assert_array_equal(dense.cpu().numpy(), ref)


@pytest.mark.parametrize("dyadic", [True, False])
def test_run_leiden_multilevel_matches_oracle(device, dyadic):
    src, dst, w = lg.planted(31, 3, 1500, 40, edges_per_vertex=6.0, dyadic=dyadic, isolated=9)
    print(f"run_leiden multilevel dyadic={dyadic}", flush=True)
    s, d, x = _dev(device, src, dst, w)
    vertex, part, q = algorithm.run_leiden(s, d, x, G=3, seq_len=1500, max_inner_iter=8, seed=2)
    rv, rp, rq = L.run_leiden(src, dst, w, graphs=3, seq_len=1500, max_inner_iter=8, seed=2)
    np.testing.assert_array_equal(vertex.cpu().numpy(), rv)
    np.testing.assert_array_equal(part.cpu().numpy(), rp)
    assert q == pytest.approx(rq, abs=1e-9)


def test_ring_of_cliques_end_to_end(device):
    src, dst, w, S = lg.ring_of_cliques(2, 6, 5, seq_len=34)
    s, d, x = _dev(device, src, dst, w)
    vertex, part, q = algorithm.run_leiden(s, d, x, G=2, seq_len=S)
    by_clique = part.cpu().numpy().reshape(2, 6, 5)
    assert (by_clique == by_clique[..., :1]).all() and np.unique(by_clique[..., 0]).size == 12


@pytest.mark.parametrize("aggregation", ["query_group", "per_query_head", "layer_wise"])
def test_partition_graphs_matches_oracle_pipeline(device, aggregation):
    """Top-k prefill edges -> build_adjacency -> Leiden -> dense community ids
    (partition.py:289-353), against the oracle's composition; then
    build_partitioned_layer (538-618) on the same edges: community count over
    all positions (sink singletons included) and the token table."""
    from community_kv_amd.graph import partition as P
    from oracle import ckv_oracle as co

    rng = np.random.default_rng(17)
    Hq, Hkv, S, sinks, kappa = 8, 2, 1200, 4, 8
    rows = S - sinks - kappa + 1
    comm = rng.integers(0, 25, S)
    idx = np.empty((Hq, rows, kappa), np.int32)
    for r in range(rows):
        p = sinks + kappa - 1 + r
        pool = np.nonzero(comm[sinks:p + 1] == comm[p])[0] + sinks
        pool = pool if pool.size >= kappa else np.arange(sinks, p + 1)
        for h in range(Hq):
            idx[h, r] = rng.choice(pool, kappa, replace=False)
    sc = (rng.integers(1, 32, idx.shape) / 32.0).astype(np.float32)
    print(f"partition_graphs pipeline {aggregation}", flush=True)
    ti, ts = torch.from_numpy(idx).to(device), torch.from_numpy(sc).to(device)
    res = P.partition_graphs(ti, ts, aggregation=aggregation, num_kv_heads=Hkv, prefill_seq_len=S, num_sink=sinks,
                             lam=0.5, leiden_resolution=1.0, leiden_seed=0)
    gi, gs, pos = P._reshape_by_aggregation(torch.from_numpy(idx), torch.from_numpy(sc), aggregation=aggregation,
                                            num_kv_heads=Hkv, num_sink=sinks)
    graphs = gi.shape[0]
    src, dst, w = co.build_adjacency(gi.numpy(), gs.numpy(), pos.numpy(), seq_len=S, lam=0.5)
    ids, q = L.partition_labels(src, dst, w, graphs=graphs, seq_len=S, resolution=1.0, max_inner_iter=3, seed=0)
    np.testing.assert_array_equal(res.community_ids.cpu().numpy(), ids)
    assert res.community_counts.cpu().tolist() == (ids.max(axis=1) + 1).tolist()
    assert res.modularity == pytest.approx(q, abs=1e-9)
    keys = torch.randn(Hkv, S, 128, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(device)
    layer = P.build_partitioned_layer(layer_idx=0, topk_indices=ti, topk_scores=ts, keys=keys, num_sink=sinks,
                                      lam=0.5, leiden_resolution=1.0, leiden_seed=0, max_decode_tokens=4,
                                      aggregation=aggregation)
    assert layer.community_counts.cpu().tolist() == (ids.max(axis=1) + 1).tolist()
    np.testing.assert_array_equal(layer.token_communities[:, :S].cpu().numpy(), ids)
    assert (layer.token_communities[:, S:] == -1).all()


def test_build_adjacency_known_answers(device):
    """The reference tests' coalescing / discard cases (test_partition.py:212-250) through ckv_build_adjacency."""
    import json
    import os

    from community_kv_amd.graph.partition import build_adjacency

    golden = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))
    for name in ("adjacency_coalesces", "adjacency_discards_outside"):
        ka = golden[name]
        src, dst, w = build_adjacency(torch.tensor(ka["indices"], dtype=torch.int32, device=device),
                                      torch.tensor(ka["scores"], dtype=torch.float32, device=device),
                                      torch.tensor(ka["query_positions"], dtype=torch.int64, device=device),
                                      seq_len=ka["seq_len"], lam=ka["lam"])
        got = sorted(zip(src.tolist(), dst.tolist(), w.tolist()))
        assert got == sorted(tuple(p) for p in ka["pairs"]), name


@pytest.mark.parametrize("lam,dyadic", [(0.5, True), (1.0, False), (0.0, True), (0.3, False)])
def test_build_adjacency_matches_oracle(device, lam, dyadic):
    from community_kv_amd.graph.partition import build_adjacency
    from oracle import ckv_oracle as co

    rng = np.random.default_rng(int(lam * 10) + dyadic)
    G, R, kappa, S = 3, 2000, 8, 1500
    idx = rng.integers(0, S, (G, R, kappa)).astype(np.int32)
    idx[rng.random(idx.shape) < 0.05] = -1
    idx[rng.random(idx.shape) < 0.02] = S + 5
    sc = (rng.integers(1, 32, idx.shape) / 32.0 if dyadic else rng.random(idx.shape)).astype(np.float32)
    pos = rng.integers(0, S, (G, R)).astype(np.int64)
    print(f"build_adjacency lam={lam} dyadic={dyadic}", flush=True)
    s, d, w = build_adjacency(*_dev(device, idx, sc, pos), seq_len=S, lam=lam)
    rs, rd, rw = co.build_adjacency(idx, sc, pos, seq_len=S, lam=lam)
    np.testing.assert_array_equal(s.cpu().numpy(), rs)
    np.testing.assert_array_equal(d.cpu().numpy(), rd)
    if dyadic:
        np.testing.assert_array_equal(w.cpu().numpy(), rw)
    else:
        np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6)


def test_run_leiden_rejects_edges_across_graphs(device):
    s, d, w = _dev(device, np.array([0, 3], np.int32), np.array([1, 5], np.int32), np.ones(2, np.float32))
    with pytest.raises(ValueError, match="same graph"):
        algorithm.run_leiden(s, d, w, G=2, seq_len=4)


def test_overflow_raised_during_local_moving_reaches_the_caller(device):
    """A table overflow flagged by the local-moving sweeps must survive the
    refinement's control reset and make run_leiden raise (the hook raises the
    device flag after local moving, as a broken table bound would)."""
    from community_kv_amd import _native

    src, dst, w = lg.planted(3, 2, 300, 6)
    s, d, x = _dev(device, src, dst, w)
    print("overflow flag after local moving", flush=True)
    lib = _native.lib()
    lib.ckv_leiden_test_raise_overflow(1)
    try:
        with pytest.raises(RuntimeError, match="overflowed"):
            algorithm.run_leiden(s, d, x, G=2, seq_len=300)
    finally:
        lib.ckv_leiden_test_raise_overflow(0)
    torch.cuda.synchronize()
    _vertex, _part, q = algorithm.run_leiden(s, d, x, G=2, seq_len=300)
    assert np.isfinite(q)
