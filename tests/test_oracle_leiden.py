"""Pins the Leiden oracle (oracle/leiden.py): the reference tests' known
answers, the gain formula against modularity differences from the textbook
definition, convergence and refinement invariants, a closed-form optimum and
the aggregation invariance.  CPU only."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
from scipy.sparse import coo_matrix
from scipy.sparse.csgraph import connected_components

from oracle import leiden as L
from tests import _leiden_graphs as lg

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def _dense_adjacency(src, dst, w, V):
    A = np.zeros((V, V))
    for s, d, x in zip(src, dst, w.astype(np.float64)):
        A[s, d] += x
        A[d, s] += x  # a self loop lands twice on the diagonal: A_ii = 2w
    return A


def _textbook_q(A, labels, resolution=1.0):
    """Q = 1/2m sum_ij (A_ij - gamma k_i k_j / 2m) delta(c_i, c_j)."""
    k = A.sum(axis=1)
    two_m = k.sum()
    same = labels[:, None] == labels[None, :]
    return float(((A - resolution * np.outer(k, k) / two_m) * same).sum() / two_m)


def test_densify_known_answer():
    ka = GOLDEN["leiden_densify"]
    dense, width = L.densify_per_graph(np.asarray(ka["labels"]), ka["G"], ka["seq_len"])
    assert dense.tolist() == ka["dense"] and width == ka["width"]


def test_two_component_modularity_known_answer():
    ka = GOLDEN["leiden_two_component_modularity"]
    q = L.disjoint_modularity(ka["src"], ka["dst"], np.asarray(ka["weight"], np.float32), ka["labels"],
                              ka["resolution"])
    assert q == pytest.approx(ka["modularity"], abs=1e-12)


def test_pcg_hash_matches_scalar_definition():
    def scalar(x):
        state = (x * 747796405 + 2891336453) & 0xFFFFFFFF
        word = (((state >> ((state >> 28) + 4)) ^ state) * 277803737) & 0xFFFFFFFF
        return ((word >> 22) ^ word) & 0xFFFFFFFF

    xs = np.array([0, 1, 2, 12345, 2**31 - 1, 2**32 - 1], dtype=np.uint64)
    assert L.pcg_hash(xs).tolist() == [scalar(int(x)) for x in xs]
    u = L.rand_uniform(np.arange(1000) % 3, np.arange(1000), 0, 2, 7)
    assert u.dtype == np.float32 and (u >= 0).all() and (u < 1).all()


@pytest.mark.parametrize("resolution", [1.0, 0.5, 2.0])
def test_gain_equals_textbook_modularity_difference(resolution):
    src, dst, w = lg.planted(3, 1, 60, 4, self_loops=3, dyadic=False)
    csr = L.build_csr(src, dst, w, 1, 60)
    A = _dense_adjacency(src, dst, w, 60)
    rng = np.random.default_rng(1)
    labels = rng.integers(0, 8, 60).astype(np.int32)  # communities named by member-vertex ids below
    labels = np.asarray([np.nonzero(labels == l)[0][0] for l in labels], np.int32)
    v, c, dq = L.move_gains(csr, labels, L.sigma_tot(csr, labels), resolution)
    assert v.size > 50
    q0 = _textbook_q(A, labels, resolution)
    for i in rng.choice(v.size, 40, replace=False):
        moved = labels.copy()
        moved[v[i]] = c[i]
        # gains use float32 neighbour weights: agree to float rounding
        assert dq[i] == pytest.approx(_textbook_q(A, moved, resolution) - q0, abs=2e-6)


def test_modularity_per_graph_matches_textbook():
    src, dst, w = lg.planted(5, 2, 50, 3, self_loops=2, dyadic=False)
    csr = L.build_csr(src, dst, w, 2, 50)
    labels = np.random.default_rng(0).integers(0, 4, 100).astype(np.int32) + (np.arange(100) // 50) * 50
    q = L.modularity_per_graph(csr, labels, 1.0)
    for g in range(2):
        keep = (src // 50) == g
        A = _dense_adjacency(src[keep] - 50 * g, dst[keep] - 50 * g, w[keep], 50)
        assert q[g] == pytest.approx(_textbook_q(A, labels[50 * g:50 * g + 50]), abs=1e-9)


def test_local_moving_converges_and_refinement_refines():
    src, dst, w = lg.planted(11, 2, 300, 6, isolated=5)
    labels, _, parent = L.batched_leiden(src, dst, w, graphs=2, seq_len=300, max_inner_iter=64, return_stages=True)
    csr = L.build_csr(src, dst, w, 2, 300)
    lm = np.where(parent < 0, np.arange(600), parent).astype(np.int32)
    v, c, dq = L.move_gains(csr, lm, L.sigma_tot(csr, lm), 1.0)
    assert dq.max() < 1e-6  # converged in both directions: no move gains more than the jitter scale
    edge = labels >= 0
    assert (labels[~edge] == -1).all() and (np.diff(csr.row_ptr)[~edge] == 0).all()
    # every refined community lies inside one local-moving community and is connected
    for r in np.unique(labels[edge]):
        members = np.nonzero(labels == r)[0]
        assert np.unique(parent[members]).size == 1
        keep = np.isin(src, members) & np.isin(dst, members)
        idx = {m: i for i, m in enumerate(members)}
        a = coo_matrix((np.ones(keep.sum()), ([idx[s] for s in src[keep]], [idx[d] for d in dst[keep]])),
                       shape=(members.size, members.size))
        assert connected_components(a, directed=False)[0] == 1


def test_ring_of_cliques_recovers_cliques_with_closed_form_modularity():
    cliques, size = 6, 5
    src, dst, w, S = lg.ring_of_cliques(2, cliques, size, seq_len=34)
    vertex, part, q = L.run_leiden(src, dst, w, graphs=2, seq_len=S)
    assert vertex.tolist() == [g * S + i for g in range(2) for i in range(cliques * size)]
    by_clique = part.reshape(2, cliques, size)
    assert (by_clique == by_clique[..., :1]).all()
    assert np.unique(by_clique[..., 0]).size == 2 * cliques
    # union of two copies: the in-weight fraction is that of one copy, the
    # degree term halves (twice the communities, four times (2m)^2)
    m = cliques * (size * (size - 1) / 2 + 1)
    expected = cliques * (size * (size - 1) / 2) / m - cliques * ((size * (size - 1) + 2) / (2 * m)) ** 2 / 2
    assert q == pytest.approx(expected, abs=1e-12)


def test_aggregation_preserves_modularity_and_weight():
    src, dst, w = lg.planted(21, 2, 200, 5, self_loops=4, dyadic=True)
    lab, _ = L.batched_leiden(src, dst, w, graphs=2, seq_len=200)
    lab = np.where(lab < 0, np.arange(400), lab).astype(np.int32)
    dense, width = L.densify_per_graph(lab, 2, 200)
    s2, d2, w2 = L.aggregate_coo(src, dst, w, dense, 2 * width)
    assert (s2 <= d2).all() and np.unique(s2.astype(np.int64) * 2 * width + d2).size == s2.size
    assert float(w2.astype(np.float64).sum()) == float(w.astype(np.float64).sum())
    q_orig = L.disjoint_modularity(src, dst, w, dense, 1.0)
    q_agg = L.disjoint_modularity(s2, d2, w2, np.arange(2 * width), 1.0)
    assert q_agg == pytest.approx(q_orig, abs=1e-12)


def test_hub_table_cap_keeps_first_communities():
    src, dst, w, S = lg.hub(2, 1500, 40)
    csr = L.build_csr(src, dst, w, 1, S)
    labels = np.arange(S, dtype=np.int32)
    v, c, _ = L.move_gains(csr, labels, L.sigma_tot(csr, labels), 1.0)
    hub_c = np.sort(c[v == 0])
    assert hub_c.size == L.TABLE_CAP and hub_c.tolist() == list(range(1, L.TABLE_CAP + 1))


def test_fill_and_dense_remap():
    m = np.array([[5, -1, 5, 2, -1], [-1, -1, 0, 0, 7]])
    filled = L.fill_isolated(m)
    assert filled.tolist() == [[5, 6, 5, 2, 7], [8, 9, 0, 0, 7]]
    assert L.dense_remap(filled).tolist() == [[1, 2, 1, 0, 3], [2, 3, 0, 0, 1]]


def test_boltzmann_refinement_samples_softmax_of_gains():
    """Gumbel-max (refinement.cu:195-245): over independent draws the chosen
    target follows P(c) ∝ exp(dQ_c / theta) over the non-negative-gain
    candidates and staying (dQ = 0)."""
    # vertex 0 joined to triangle {1,2,3} (edges 1) by two edges of 1 and to
    # triangle {4,5,6} (edges 0.5) by two edges of 0.8; a separate triangle
    # {7,8,9}; one parent community; vertices 1..9 already grouped
    src = np.array([0, 0, 1, 1, 2, 0, 0, 4, 4, 5, 7, 8, 7])
    dst = np.array([1, 2, 2, 3, 3, 4, 5, 5, 6, 6, 8, 9, 9])
    w = np.array([1, 1, 1, 1, 1, 0.8, 0.8, 0.5, 0.5, 0.5, 1, 1, 1], np.float32)
    csr = L.build_csr(src, dst, w, 1, 10)
    labels = np.array([0, 1, 1, 1, 4, 4, 4, 7, 7, 7], np.int32)
    parent = np.zeros(10, np.int32)
    sig = L.sigma_tot(csr, labels)
    v, c, dq = L.move_gains(csr, labels, sig, 1.0)
    gains = {int(cc): float(d) for vv, cc, d in zip(v, c, dq) if vv == 0}
    assert gains[1] > 0 and gains[4] > 0 and set(gains) == {1, 4}
    theta = 0.02
    counts = {0: 0, 1: 0, 4: 0}
    draws = 4000
    for sweep in range(draws):
        prop, _ = L.refine_propose(csr, parent, labels, sig, L.sigma_tot(csr, parent), resolution=1.0,
                                   theta=theta, boltzmann=True, level=1, sweep=sweep % 65536, seed=sweep // 65536)
        counts[int(prop[0])] += 1
    logits = np.array([0.0, gains[1], gains[4]]) / theta
    p = np.exp(logits - logits.max())
    p /= p.sum()
    freq = np.array([counts[0], counts[1], counts[4]]) / draws
    np.testing.assert_allclose(freq, p, atol=0.03)
