"""Prefill attention + top-kappa edge export on the GPU against the oracle
(oracle/prefill.py): small sequences checked row by row in full, and the
Qwen3-8B 32k configuration checked on sampled rows (each row's oracle costs
O(S * D))."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from community_kv_amd.attention.flash_attention import prefill_attention_topk
from oracle import prefill as op

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-2     # bf16 output, max-abs
LSE_TOL = 1e-4
VAL_RTOL = 1e-3    # reference probability of the quantised score


def _random_qkv(S, Hq, Hkv, seed, device, *, coarse=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, S, Hq, 128, generator=g)
    k = torch.randn(1, S, Hkv, 128, generator=g)
    v = torch.randn(1, S, Hkv, 128, generator=g)
    if coarse:
        # multiples of 1/4 in [-2, 2]: every q.k is exact in float32 whatever
        # the accumulation order, and quantised ties are frequent
        q = (q * 2).round().clamp(-8, 8) / 4
        k = (k * 2).round().clamp(-8, 8) / 4
    else:
        q = q * 0.4
        k = k * 0.4
    return (q.to(torch.bfloat16).to(device), k.to(torch.bfloat16).to(device), v.to(torch.bfloat16).to(device))


def _check_rows(q, k, v, res, rows, heads, *, scale, num_sink, kappa, exact_sets, raw=False):
    out, lse, _, _, tv, ti = res
    qn = q[0].float().cpu().numpy()
    kn = k[0].float().cpu().numpy()
    vn = v[0].float().cpu().numpy()
    ref = op.prefill_rows(qn, kn, vn, rows, heads, softmax_scale=scale, num_sink=num_sink, kappa=kappa)
    out_g = out[0].float().cpu().numpy()
    lse_g = lse[0].cpu().numpy()
    tv_g = tv[0].cpu().numpy()
    ti_g = ti[0].cpu().numpy()
    skip = op.topk_row_skip(num_sink, kappa)
    for i, (r, h) in enumerate(zip(rows, heads)):
        case = f"row {r} head {h}"
        assert abs(lse_g[h, r] - ref["lse"][i]) < LSE_TOL, case
        assert np.abs(out_g[r, h] - ref["out"][i]).max() < OUT_TOL, case
        if r < skip:
            continue
        got = ti_g[h, r - skip]
        if exact_sets:
            assert got.tolist() == ref["topk_idx"][i].tolist(), case
        else:
            ok, msg = op.consistent_topk(ref["raw"][i], got, num_sink=num_sink, row=r, kappa=kappa)
            assert ok, f"{case}: {msg}"
        keys = op.quantise_score(ref["raw"][i][got].astype(np.float32))
        if raw:
            want = op.dequantise_key(keys).astype(np.float64)
            np.testing.assert_allclose(tv_g[h, r - skip], want, atol=1e-6, err_msg=case)
        else:
            want = np.exp(op.dequantise_key(keys).astype(np.float64) * scale - ref["lse"][i])
            np.testing.assert_allclose(tv_g[h, r - skip], want, rtol=VAL_RTOL, atol=1e-9, err_msg=case)
        if exact_sets:
            # descending (quantised score, column) order
            assert np.all(np.diff(op.pack_candidates(keys, got)) < 0), case


SMALL = [
    # S, Hq, Hkv, num_sink, kappa, coarse
    (200, 4, 1, 10, 8, False),
    (333, 8, 8, 0, 16, False),
    (130, 8, 2, 3, 4, True),
    (257, 6, 2, 10, 8, True),    # G = 3: packed rows straddle positions
    (64, 4, 4, 10, 8, True),
    (20, 4, 1, 10, 16, False),   # fewer rows than the skip: empty top-k output
    # long rows of tied coarse scores: the pending candidates are merged into
    # the queues many times per row (queue sizes 8 and 4)
    (1536, 8, 2, 10, 8, True),
    (1024, 4, 1, 0, 4, True),
]


@pytest.mark.parametrize("S,Hq,Hkv,num_sink,kappa,coarse", SMALL)
def test_prefill_small_matches_oracle(device, S, Hq, Hkv, num_sink, kappa, coarse):
    print(f"prefill S={S} Hq={Hq} Hkv={Hkv} sinks={num_sink} kappa={kappa} coarse={coarse}", flush=True)
    q, k, v = _random_qkv(S, Hq, Hkv, seed=S + kappa, device=device, coarse=coarse)
    scale = 128 ** -0.5
    res = prefill_attention_topk(q, k, v, softmax_scale=scale, num_sink=num_sink, kappa=kappa)
    torch.cuda.synchronize()
    skip = op.topk_row_skip(num_sink, kappa)
    assert res[4].shape == (1, Hq, max(0, S - skip), kappa)
    rows = np.repeat(np.arange(S), Hq)
    heads = np.tile(np.arange(Hq), S)
    _check_rows(q, k, v, res, rows, heads, scale=scale, num_sink=num_sink, kappa=kappa, exact_sets=coarse)


def test_prefill_raw_scores(device):
    print("prefill raw scores", flush=True)
    q, k, v = _random_qkv(150, 4, 2, seed=9, device=device, coarse=True)
    res = prefill_attention_topk(q, k, v, softmax_scale=0.1, num_sink=2, kappa=8, raw_scores=True)
    torch.cuda.synchronize()
    rows = np.repeat(np.arange(150), 4)
    heads = np.tile(np.arange(4), 150)
    _check_rows(q, k, v, res, rows, heads, scale=0.1, num_sink=2, kappa=8, exact_sets=True, raw=True)


def test_prefill_rejects_bad_arguments(device):
    q, k, v = _random_qkv(64, 4, 2, seed=1, device=device)
    with pytest.raises(RuntimeError):
        prefill_attention_topk(q, k, v, softmax_scale=0.1, num_sink=2, kappa=17)
    with pytest.raises(RuntimeError):
        prefill_attention_topk(q, k, v, softmax_scale=-1.0, num_sink=2, kappa=8)


def test_prefill_config5_sampled_rows(device):
    """Qwen3-8B layer shape at 32k with planted clusters, kappa 16: 96 sampled
    (row, head) pairs plus the first and last eligible rows against the oracle,
    and size-independent properties over every row."""
    import bench

    print("prefill config 5 (S=32768, 32/8 heads, kappa 16)", flush=True)
    q, k, v = bench.planted_prefill_inputs(device)
    S, Hq = q.shape[1], q.shape[2]
    kappa, sinks = 16, 10
    scale = 128 ** -0.5
    res = prefill_attention_topk(q, k, v, softmax_scale=scale, num_sink=sinks, kappa=kappa)
    torch.cuda.synchronize()
    out, lse, _, _, tv, ti = res
    skip = op.topk_row_skip(sinks, kappa)
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    # every row: indices distinct, inside [sinks, row], values in (0, 1], sorted descending
    idx = ti[0].long()
    rows_t = torch.arange(skip, S, device=device).view(1, -1, 1)
    assert bool((idx >= sinks).all()) and bool((idx <= rows_t).all())
    srt = idx.sort(dim=-1).values
    assert bool((srt[..., 1:] != srt[..., :-1]).all())
    assert bool((tv[0] > 0).all()) and bool((tv[0] <= 1.0 + 1e-6).all())
    assert bool((tv[0][..., 1:] <= tv[0][..., :-1]).all())
    rng = np.random.default_rng(5)
    rows = np.r_[rng.integers(skip, S, 96), skip, S - 1, S - 1, 0]
    heads = np.r_[rng.integers(0, Hq, 96), 0, 0, Hq - 1, 3]
    _check_rows(q, k, v, res, rows, heads, scale=scale, num_sink=sinks, kappa=kappa, exact_sets=False)


@pytest.mark.parametrize("kappa", [16, 8])
def test_prefill_config5_coarse_grid_exact_sets(device, kappa):
    """Config 5's full shape (32,768 tokens, 32/8 heads; kappa 16, and the
    reference's width 8) with the planted inputs moved onto a coarse grid: q
    and k rounded to multiples of 1/64 in [-1, 1] (at most 6 significant bits,
    so every product is a multiple of 2^-12 and every partial sum of 128 of
    them is exact in float32 whatever the MMA's accumulation order).  Index
    sets and their order must then be bit-identical to the oracle's exact
    top-kappa on 1,000 sampled (row, head) pairs plus the first and last
    eligible rows of several heads."""
    import bench

    print(f"prefill config 5 coarse grid (S=32768, 32/8 heads, kappa {kappa}, exact sets)", flush=True)
    q, k, v = bench.planted_prefill_inputs(device)
    q = ((q.float() * 64).round().clamp(-64, 64) / 64).to(torch.bfloat16)
    k = ((k.float() * 64).round().clamp(-64, 64) / 64).to(torch.bfloat16)
    S, Hq = q.shape[1], q.shape[2]
    sinks = 10
    scale = 128 ** -0.5
    res = prefill_attention_topk(q, k, v, softmax_scale=scale, num_sink=sinks, kappa=kappa)
    torch.cuda.synchronize()
    skip = op.topk_row_skip(sinks, kappa)
    rng = np.random.default_rng(17 + kappa)
    rows = np.r_[rng.integers(skip, S, 1000), [skip] * 4, [S - 1] * 4]
    heads = np.r_[rng.integers(0, Hq, 1000), 0, 7, 16, Hq - 1, 0, 9, 22, Hq - 1]
    _check_rows(q, k, v, res, rows, heads, scale=scale, num_sink=sinks, kappa=kappa, exact_sets=True)
