"""Pins the oracle's bit-level numerics against numpy/torch and the mathematics."""

from __future__ import annotations

import numpy as np
import torch

from oracle import ckv_oracle as co
from oracle import numerics as nm


def _sample_floats(n=200_000, seed=0):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    extra = np.array([0.0, -0.0, 1.0, -1.0, 448.0, 464.0, 480.0, -500.0, 2**-9, 2**-10, 3 * 2**-10,
                      1e-30, 65504.0, 65520.0, 1e6, np.inf, -np.inf], np.float32)
    return np.concatenate([x, extra, rng.standard_normal(n).astype(np.float32) * 10])


def test_bf16_rounding_matches_torch():
    x = _sample_floats()
    ours = nm.f32_to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_fp16_key_matches_torch_cast():
    x = _sample_floats()
    ours = nm.f32_to_f16_bits(x)
    ref = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_e4m3_matches_torch_after_clamp():
    x = _sample_floats()
    clamped = np.clip(x, -448.0, 448.0).astype(np.float32)
    ref = torch.from_numpy(clamped).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    ours = nm.f32_to_e4m3(x)
    # signed zero: torch keeps the sign of zero as well
    assert np.array_equal(ours, ref)
    table_ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(nm.E4M3_TABLE), np.isnan(table_ref))
    fin = ~np.isnan(table_ref)
    assert np.array_equal(nm.E4M3_TABLE[fin], table_ref[fin])


def test_ckv_exp_is_accurate():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-100, 0, 200_000), rng.uniform(-1, 1, 100_000),
                        rng.uniform(0, 80, 10_000)]).astype(np.float32)
    ours = nm.ckv_exp(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    normal = ref > 2.0 ** -125
    rel = np.abs(ours[normal] - ref[normal]) / ref[normal]
    assert rel.max() < 4 * 2.0 ** -24
    assert nm.ckv_exp(np.float32(0.0)) == 1.0
    assert nm.ckv_exp(np.float32(-np.inf)) == 0.0
    assert nm.ckv_exp(np.float32(-200.0)) == 0.0


def test_ckv_log_is_accurate():
    rng = np.random.default_rng(2)
    x = np.exp(rng.uniform(0, 60, 200_000)).astype(np.float32)
    x = np.concatenate([x, np.array([1.0, 2.0, 1.4142135, 1.4142137], np.float32)])
    ours = nm.ckv_log(x).astype(np.float64)
    ref = np.log(x.astype(np.float64))
    err = np.abs(ours - ref) / np.maximum(np.abs(ref), 1.0)
    assert err.max() < 4 * 2.0 ** -24
    assert nm.ckv_log(np.float32(1.0)) == 0.0


def test_pinned_dot_is_exact_for_bf16_by_fp8_products():
    """bf16 x e4m3 products are exact in fp32, so any summation order of small
    integers is exact; with real data the pinned order must stay within fp32
    rounding of the float64 dot."""
    rng = np.random.default_rng(4)
    q = nm.f32_to_bf16(rng.integers(-8, 8, size=(5, 128)).astype(np.float32))
    c = nm.e4m3_to_f32(nm.f32_to_e4m3(rng.integers(-8, 8, size=(5, 128)).astype(np.float32)))
    assert np.array_equal(co.pinned_dot16x8(q, c), (q.astype(np.float64) * c).sum(-1).astype(np.float32))
    q = nm.f32_to_bf16(rng.standard_normal((1000, 128)).astype(np.float32))
    c = nm.e4m3_to_f32(nm.f32_to_e4m3(rng.standard_normal((1000, 128)).astype(np.float32)))
    ref = (q.astype(np.float64) * c).sum(-1)
    got = co.pinned_dot16x8(q, c)
    assert np.max(np.abs(got - ref)) < 1e-4


def test_blocked_community_sums_order():
    """Centroid sums: a scalar loop over each community's members (ascending
    positions, blocks of 64 from +0, block sums in order from +0) agrees bit
    for bit; communities of at most 64 members equal the plain in-order sum;
    every sum is within fp32 rounding of the float64 sum."""
    rng = np.random.default_rng(11)
    n, cap = 3000, 12
    w = 1.0 / np.arange(1, cap + 1) ** 1.5
    ids = rng.choice(cap, size=n, p=w / w.sum())
    ids[ids == 7] = 8  # an empty community
    rows = (rng.standard_normal((n, 3)) * np.exp(2 * rng.standard_normal((n, 1)))).astype(np.float32)
    got = co.blocked_community_sums(ids, rows, cap)
    for c in range(cap):
        mem = rows[ids == c]
        total = np.zeros(3, np.float32)
        for b0 in range(0, len(mem), 64):
            blk = np.zeros(3, np.float32)
            for x in mem[b0:b0 + 64]:
                blk = (blk + x).astype(np.float32)
            total = (total + blk).astype(np.float32)
        assert np.array_equal(got[c], total), c
        ref = mem.astype(np.float64).sum(0)
        assert np.all(np.abs(got[c] - ref) <= 1e-5 * np.abs(mem).sum(0) + 1e-30)
        if len(mem) <= 64:
            seq = np.zeros((1, 3), np.float32)
            np.add.at(seq, np.zeros(len(mem), np.int64), mem)  # scatter_add_'s in-order CPU sum
            assert np.array_equal(got[c], seq[0])
    assert not got[7].any()
    assert (np.bincount(ids, minlength=cap) > 64).sum() >= 2  # the blocked path is exercised


def test_attention_matches_torch_sdpa():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((4, 128)).astype(np.float32)
    k = rng.standard_normal((300, 128)).astype(np.float32)
    v = rng.standard_normal((300, 128)).astype(np.float32)
    pos = rng.permutation(300)[:130].astype(np.int32)
    pos = np.concatenate([pos, -np.ones(62, np.int32)])
    out, lse, _ = co.attend(q, k, v, pos, 0.125)
    sel = pos[pos >= 0]
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).double()[None, :, None, :].transpose(1, 2),
        torch.from_numpy(k[sel]).double()[None, None],
        torch.from_numpy(v[sel]).double()[None, None], scale=0.125)
    assert np.allclose(out, ref[0, 0].numpy(), atol=1e-12)
    s = (q.astype(np.float64) @ k[sel].T.astype(np.float64)) * 0.125
    assert np.allclose(lse, np.log(np.exp(s).sum(1)), atol=1e-12)


def test_topk_candidates_break_ties_by_position():
    scores = np.array([-np.inf, 1.0, 3.0, 3.0, 2.0, 3.0, 0.5, 7.0, 1.0, 1.0, 1.0])
    pos = np.array([0, 50, 40, 20, 30, 10, 60, 70, 5, 4, -1], np.int32)
    sc, ps = co.topk_candidates(scores, pos, num_sink=1, kappa=8)
    assert ps.tolist() == [70, 10, 20, 40, 30, 4, 5, 50]
