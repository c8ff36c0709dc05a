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
