"""Pins the prefill oracle (oracle/prefill.py) against closed forms, a brute-force
sort and scipy's softmax; none of these retypes the oracle's own formula."""

from __future__ import annotations

import numpy as np
import pytest
from scipy.special import logsumexp, softmax

from oracle import prefill as op


def test_quantiser_closed_form_values():
    # (s + 48) * 256 at exact binary points, the clamp ends and round-half-even.
    s = np.array([-48.0, 0.0, 1.0, -1.0, 79.99609375, 80.0, 200.0, -60.0, -np.inf,
                  -48.0 + 0.5 / 256, -48.0 + 1.5 / 256, 0.25 / 256], np.float32)
    want = [0, 12288, 12544, 12032, 32767, 32767, 32767, 0, 0, 0, 2, 12288]
    assert op.quantise_score(s).tolist() == want


def test_dequantise_inverts_quantise_on_grid():
    keys = np.arange(0, 32768, 7)
    assert np.array_equal(op.quantise_score(op.dequantise_key(keys)), keys)


def test_skip_matches_reference_row_count():
    # community-kv.patch:69-76: skip = seqlen_q + sinks + 7 - seqlen_k for kTopK = 8.
    for sinks in (0, 1, 10):
        assert op.topk_row_skip(sinks, 8) == sinks + 7


def _inputs(S, Hq, Hkv, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((S, Hq, 128)) * scale).astype(np.float32)
    k = (rng.standard_normal((S, Hkv, 128)) * scale).astype(np.float32)
    v = rng.standard_normal((S, Hkv, 128)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("num_sink,kappa", [(0, 8), (10, 8), (3, 16)])
def test_topk_matches_brute_force_sort(num_sink, kappa):
    S, Hq, Hkv = 70, 4, 2
    q, k, v = _inputs(S, Hq, Hkv, seed=kappa + num_sink, scale=0.3)
    # Coarsen scores so quantised ties are frequent and the column tie rule matters.
    k = np.round(k * 4) / 4
    scale = 1 / np.sqrt(128)
    out, lse, tv, ti, res = op.prefill_attention_topk(q, k, v, softmax_scale=scale, num_sink=num_sink, kappa=kappa)
    skip = num_sink + kappa - 1
    assert ti.shape == (Hq, S - skip, kappa)
    ties = 0
    for h in range(Hq):
        for r in range(skip, S):
            s = (k[:r + 1, h // 2].astype(np.float64) @ q[r, h].astype(np.float64))
            cand = []
            for c in range(num_sink, r + 1):
                key = int(np.clip(np.rint(np.float32(np.float32(s[c]) + np.float32(48)) * np.float32(256)), 0, 32767))
                cand.append((key, c))
            cand.sort(reverse=True)
            want = [c for _, c in cand[:kappa]]
            keys = [kk for kk, _ in cand]
            ties += len(keys) - len(set(keys))
            assert ti[h, r - skip].tolist() == want
            lse_ref = logsumexp(s * scale)
            vals = [np.exp((kk / 256 - 48) * scale - lse_ref) for kk, _ in cand[:kappa]]
            np.testing.assert_allclose(tv[h, r - skip], vals, rtol=1e-6)
    assert ties > 0


def test_attention_half_matches_scipy_softmax():
    S, Hq, Hkv = 50, 8, 2
    q, k, v = _inputs(S, Hq, Hkv, seed=5)
    scale = 0.088
    out, lse, *_ = op.prefill_attention_topk(q, k, v, softmax_scale=scale, num_sink=4, kappa=8)
    g = Hq // Hkv
    for h in range(Hq):
        for r in range(S):
            s = k[:r + 1, h // g].astype(np.float64) @ q[r, h].astype(np.float64) * scale
            np.testing.assert_allclose(lse[h, r], logsumexp(s), rtol=1e-12)
            np.testing.assert_allclose(out[r, h], softmax(s) @ v[:r + 1, h // g].astype(np.float64), rtol=1e-9,
                                       atol=1e-12)


def test_consistent_topk_accepts_exact_and_rejects_swaps():
    rng = np.random.default_rng(3)
    s = rng.standard_normal(300)
    row, sinks, kappa = 299, 5, 8
    keys = op.quantise_score(s[sinks:].astype(np.float32))
    cols = np.arange(sinks, row + 1)
    order = np.argsort(-op.pack_candidates(keys, cols), kind="stable")[:kappa]
    best = cols[order]
    assert op.consistent_topk(s, best, num_sink=sinks, row=row, kappa=kappa)[0]
    worse = best.copy()
    worse[-1] = cols[np.argsort(-op.pack_candidates(keys, cols))[kappa + 20]]
    assert not op.consistent_topk(s, worse, num_sink=sinks, row=row, kappa=kappa)[0]
    assert not op.consistent_topk(s, np.r_[best[:-1], 2], num_sink=sinks, row=row, kappa=kappa)[0]
    assert not op.consistent_topk(s, np.r_[best[:-1], best[0]], num_sink=sinks, row=row, kappa=kappa)[0]


# ---------------------------------------------------------------------------
# The reference's approximate top-8 (WarpSelect<2, 8, 16>, community-kv.patch:477-723)
# ---------------------------------------------------------------------------


def test_warpselect_lane_classes_are_column_pairs():
    # lane l of a quad owns columns 8j + 2l and 8j + 2l + 1
    assert op.warpselect_lane(np.arange(16)).tolist() == [0, 0, 1, 1, 2, 2, 3, 3] * 2
    assert op.warpselect_lane([130, 133, 1023]).tolist() == [1, 2, 3]


def test_warpselect_drops_the_seventh_of_one_lane():
    """Eight best columns: seven in lane 0's class (0, 1, 8, 9, 16, 17, 24) and
    column 2 (lane 1).  Lane 0 keeps only six, so its weakest (24) is replaced
    by the best remaining column of another class (column 11, lane 1)."""
    row = 40
    s = np.full(row + 1, -1.0)
    for rank, c in enumerate([0, 1, 8, 9, 16, 17, 24]):
        s[c] = 10.0 - rank            # 10, 9, ..., 4
    s[2] = 3.5
    s[11] = 2.0                       # next best outside the seven
    s[25] = 1.5                       # lane 0 again: below lane 0's sixth, and lane 0 is full
    got = op.warpselect_topk(s, row=row, num_sink=0)
    assert got.tolist() == [0, 1, 8, 9, 16, 17, 2, 11]
    exact = [0, 1, 8, 9, 16, 17, 24, 2]
    assert sorted(got.tolist()) != sorted(exact)


def test_warpselect_six_per_lane_is_exact():
    """Six of the best eight in one class still fit its queue: same set and
    order as the exact top-8."""
    row = 70
    s = np.zeros(row + 1)
    best = [64, 65, 56, 57, 48, 49, 3, 13]     # six in lane 0, then lanes 1 and 2
    for rank, c in enumerate(best):
        s[c] = 20.0 - rank
    assert op.warpselect_topk(s, row=row, num_sink=0).tolist() == best


def test_warpselect_respects_sinks_and_ties():
    """Sinks are never candidates; equal quantised scores go to the larger column."""
    row = 30
    s = np.zeros(row + 1)
    s[:4] = 50.0                      # sinks: the highest scores, excluded
    got = op.warpselect_topk(s, row=row, num_sink=4)
    # every eligible column ties: the largest columns win, at most six per lane
    want = sorted(range(4, row + 1), reverse=True)[:8]
    assert got.tolist() == want      # 30..23 covers each lane twice


@pytest.mark.parametrize("seed", range(4))
def test_warpselect_differs_only_when_a_lane_holds_seven(seed):
    """Against a brute force over random rows: the approximate set equals the
    exact top-8 exactly when no lane class holds seven or more of the exact
    eight; otherwise it holds six of that lane and the best of the rest."""
    rng = np.random.default_rng(seed)
    differ = 0
    for trial in range(300):
        row = int(rng.integers(20, 200))
        sinks = int(rng.integers(0, 8))
        s = rng.standard_normal(row + 1) * (0.02 if trial % 3 == 0 else 2.0)   # some rows full of ties
        if trial % 5 == 0:                                                       # plant a crowded lane
            cls = int(rng.integers(4))
            cols = [c for c in range(sinks, row + 1) if (c % 8) // 2 == cls]
            for c in rng.choice(cols, size=min(8, len(cols)), replace=False):
                s[c] += 6.0
        keys = op.quantise_score(s.astype(np.float32))
        cand = sorted(range(sinks, row + 1), key=lambda c: (keys[c], c), reverse=True)
        exact = cand[:8]
        per_lane = {}
        for c in exact:
            per_lane.setdefault((c % 8) // 2, []).append(c)
        crowded = [l for l, v in per_lane.items() if len(v) >= 7]
        got = op.warpselect_topk(s, row=row, num_sink=sinks).tolist()
        if not crowded:
            assert got == exact
        else:
            differ += 1
            lane = crowded[0]
            kept = [c for c in cand if (c % 8) // 2 == lane][:6]
            rest = [c for c in cand if (c % 8) // 2 != lane][:2]
            assert sorted(got) == sorted(kept + rest)
    assert differ > 0
