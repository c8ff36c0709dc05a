"""How often the reference's approximate prefill top-8 (WarpSelect<2, 8, 16>,
third_party/flash_attention/community-kv.patch:477-723, restated in
``oracle.prefill.warpselect_topk``) differs from the exact top-8 this build's
kernel emits, on config-5-shaped inputs (32,768 tokens, 32/8 heads, head_dim
128, 256 planted clusters of 128-token blocks, intra-cluster cosine 0.6,
``bench.planted_prefill_inputs``).  TEST INFRASTRUCTURE / measurement only.

    python -m oracle.warpselect_divergence [pairs] [seed]

Samples ``pairs`` (row, query head) pairs with rows past the skip, computes
each row's raw scores in float64 (quantised in float32 as the kernels do) and
prints the fraction of rows whose index sets differ, with a 95 % Wilson
interval, overall and by row range."""

from __future__ import annotations

import json
import math
import sys

import numpy as np


def wilson(k, n, z=1.96):
    if n == 0:
        return (0.0, 0.0)
    p = k / n
    den = 1 + z * z / n
    mid = (p + z * z / (2 * n)) / den
    half = z * math.sqrt(p * (1 - p) / n + z * z / (4 * n * n)) / den
    return (max(0.0, mid - half), min(1.0, mid + half))


def main(pairs=20000, seed=1, num_sink=10):
    import torch

    import bench
    from oracle import prefill as op

    q, k, _v = bench.planted_prefill_inputs(torch.device("cpu"))
    qn = q[0].float().numpy()
    kn = k[0].float().numpy()
    S, Hq = qn.shape[0], qn.shape[1]
    group = Hq // kn.shape[1]
    skip = op.topk_row_skip(num_sink, 8)
    rng = np.random.default_rng(seed)
    rows = rng.integers(skip, S, pairs)
    heads = rng.integers(0, Hq, pairs)
    bins = [(skip, 1024), (1024, 8192), (8192, S)]
    hits = {b: [0, 0] for b in bins}
    differ = 0
    crowded_lanes = 0
    for r, h in zip(rows, heads):
        s = op.row_scores(qn, kn, int(r), int(h), group)
        keys = op.quantise_score(s[num_sink:r + 1].astype(np.float32))
        packed = op.pack_candidates(keys, np.arange(num_sink, r + 1))
        exact = np.sort(packed)[::-1][:8] & ((1 << op.INDEX_BITS) - 1)
        approx = op.warpselect_topk(s, row=int(r), num_sink=num_sink)
        d = set(exact.tolist()) != set(approx.tolist())
        differ += d
        lanes = np.bincount(op.warpselect_lane(exact), minlength=4)
        crowded_lanes += int(lanes.max() >= 7)
        for b in bins:
            if b[0] <= r < b[1]:
                hits[b][0] += d
                hits[b][1] += 1
    lo, hi = wilson(differ, pairs)
    out = {"pairs": int(pairs), "rows_differing": int(differ), "fraction": differ / pairs,
           "wilson95": [lo, hi], "rows_with_a_lane_holding_7_of_8": int(crowded_lanes),
           "by_row_range": {f"[{a},{b})": {"differing": v[0], "rows": v[1]} for (a, b), v in hits.items()}}
    print(json.dumps(out))
    return out


if __name__ == "__main__":
    main(*(int(a) for a in sys.argv[1:]))
