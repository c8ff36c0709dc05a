"""CPU restatement of the prefill attention + top-kappa edge export (parity oracle).

TEST INFRASTRUCTURE ONLY.  ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` are the only callers; the product path
runs ``ckv_prefill_attention_topk`` and never imports this module.

Reference semantics (third_party/flash_attention/community-kv.patch):
  * causal attention with PackGQA: query head h reads KV head h // (Hq // Hkv)
    (patch:51-76 checks, the kernel is FlashAttention-3's forward);
  * ``softmax_lse`` is the natural log of sum_c exp(s_c * scale) over c <= row;
  * top-k rows: rows q >= num_sink + kappa - 1 (patch:69-76 with kTopK = kappa),
    candidates are columns c in [num_sink, q] (update_row, patch:574-598);
  * ranking key (patch:508-535): the raw score s = q.k is quantised as
    clamp(rint((s + 48) * 256), 0, 32767) in float32, packed above the 17-bit
    column; larger packed keys win, so equal quantised scores go to the larger
    column;
  * stored value (patch:674-678): exp((key / 256 - 48) * scale - lse).

The reference keeps six candidates per lane in four lanes and merges them
(patch:477-723), an approximation of the exact top-kappa computed here.  The
two agree unless one lane's residue class of columns holds more than six of a
row's best eight; that difference, and the FlashAttention-3 MMA rounding, are
not pinned by any fixture the reference ships (its test,
tests/community_kv/attention/test_flash_attention.py, checks keyword
arguments only).  What pins this restatement: the quantiser's closed-form
values, a brute-force sort of (key, column) pairs, and scipy's logsumexp /
softmax for the attention half (tests/test_oracle_prefill.py).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
SCORE_MIN = F32(-48.0)
SCORE_SCALE = F32(256.0)
KEY_MAX = 32767
INDEX_BITS = 17


def topk_row_skip(num_sink: int, kappa: int) -> int:
    """First row that has kappa eligible columns (patch:69-76 with equal
    query/key lengths: seqlen_q + sinks + kTopK - 1 - seqlen_k)."""
    return max(0, num_sink + kappa - 1)


def quantise_score(s) -> np.ndarray:
    """clamp(rint((s + 48) * 256), 0, 32767) evaluated in float32
    (WarpSelect::score_to_key, patch:508-512)."""
    x = np.asarray(s, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        k = ((x + SCORE_MIN * F32(-1.0)).astype(np.float32) * SCORE_SCALE).astype(np.float32)
        k = np.rint(k)
        k = np.where(np.isnan(k), 0.0, k)
    return np.clip(k, 0, KEY_MAX).astype(np.int64)


def dequantise_key(key) -> np.ndarray:
    """key / 256 - 48 in float32 (WarpSelect::key_to_score, patch:514-516)."""
    k = np.asarray(key).astype(np.float32)
    return (k / SCORE_SCALE + SCORE_MIN).astype(np.float32)


def pack_candidates(key, col) -> np.ndarray:
    """(key << 17) | col, the reference's packed ranking key (patch:518-521)."""
    return (np.asarray(key, dtype=np.int64) << INDEX_BITS) | np.asarray(col, dtype=np.int64)


def row_scores(query, key, row, head, group):
    """Raw scores q_row . k_c (float64) for c in [0, row] of query head ``head``.
    query [S, Hq, D], key [S, Hkv, D] as float arrays."""
    q = np.asarray(query[row, head], dtype=np.float64)
    k = np.asarray(key[:row + 1, head // group], dtype=np.float64)
    return k @ q


def prefill_rows(query, key, value, rows, heads, *, softmax_scale, num_sink, kappa):
    """Exact reference outputs for the listed (row, head) pairs.

    query [S, Hq, D], key/value [S, Hkv, D] (float32 arrays holding bf16 values).
    Returns dict with out [n, D] float64, lse [n], and for each pair the top
    (key, col) list (descending packed order), topk_val [n, kappa] float64,
    topk_idx [n, kappa] int64 (rows below the skip get -1 / nan), plus the raw
    float64 score vector per pair for tolerance-aware comparisons."""
    S, Hq, _ = query.shape
    Hkv = key.shape[1]
    group = Hq // Hkv
    skip = topk_row_skip(num_sink, kappa)
    n = len(rows)
    out = np.zeros((n, value.shape[-1]))
    lse = np.zeros(n)
    tk_idx = np.full((n, kappa), -1, np.int64)
    tk_key = np.full((n, kappa), -1, np.int64)
    tk_val = np.full((n, kappa), np.nan)
    raw = []
    for i, (r, h) in enumerate(zip(rows, heads)):
        s = row_scores(query, key, int(r), int(h), group)
        raw.append(s)
        z = s * float(softmax_scale)
        m = z.max()
        p = np.exp(z - m)
        l = p.sum()
        lse[i] = m + np.log(l)
        out[i] = (p @ np.asarray(value[:r + 1, h // group], dtype=np.float64)) / l
        if r >= skip:
            cols = np.arange(num_sink, r + 1)
            keys = quantise_score(s[num_sink:r + 1].astype(np.float32))
            packed = pack_candidates(keys, cols)
            order = np.argsort(-packed, kind="stable")[:kappa]
            tk_idx[i] = cols[order]
            tk_key[i] = keys[order]
            tk_val[i] = np.exp(dequantise_key(keys[order]).astype(np.float64) * float(softmax_scale) - lse[i])
    return {"out": out, "lse": lse, "topk_idx": tk_idx, "topk_key": tk_key, "topk_val": tk_val, "raw": raw}


def prefill_attention_topk(query, key, value, *, softmax_scale, num_sink, kappa):
    """Full-sequence restatement for small S: every row of every query head.
    Returns out [S, Hq, D], lse [Hq, S], topk_val/topk_idx [Hq, S - skip, kappa]."""
    S, Hq, D = query.shape
    skip = topk_row_skip(num_sink, kappa)
    rows = np.repeat(np.arange(S), Hq)
    heads = np.tile(np.arange(Hq), S)
    res = prefill_rows(query, key, value, rows, heads, softmax_scale=softmax_scale, num_sink=num_sink,
                       kappa=kappa)
    out = res["out"].reshape(S, Hq, D)
    lse = res["lse"].reshape(S, Hq).T.copy()
    nrows = max(0, S - skip)
    tv = res["topk_val"].reshape(S, Hq, kappa).transpose(1, 0, 2)[:, skip:]
    ti = res["topk_idx"].reshape(S, Hq, kappa).transpose(1, 0, 2)[:, skip:]
    assert tv.shape[1] == nrows
    return out, lse, tv.copy(), ti.copy(), res


def consistent_topk(raw_scores, chosen_cols, *, num_sink, row, kappa, eps=1e-4):
    """True when ``chosen_cols`` is the exact top-kappa set for some float32
    evaluation of the raw scores within +-eps*(1+|s|) (absorbs the MMA's
    accumulation order near a 1/256 quantisation boundary): every chosen column's
    best-case packed key must not lose to any unchosen column's worst-case key
    reversed, i.e. no unchosen column ranks strictly above a chosen one for every
    admissible rounding.  Returns (ok, message)."""
    s = np.asarray(raw_scores, dtype=np.float64)
    cols = np.arange(num_sink, row + 1)
    chosen = np.asarray(chosen_cols, dtype=np.int64)
    if len(set(chosen.tolist())) != kappa:
        return False, f"row {row}: duplicate or missing columns {chosen.tolist()}"
    if chosen.min() < num_sink or chosen.max() > row:
        return False, f"row {row}: column outside [{num_sink}, {row}]: {chosen.tolist()}"
    tol = eps * (1.0 + np.abs(s))
    hi = pack_candidates(quantise_score((s + tol).astype(np.float32)), np.arange(len(s)))
    lo = pack_candidates(quantise_score((s - tol).astype(np.float32)), np.arange(len(s)))
    mask = np.zeros(len(s), bool)
    mask[chosen] = True
    others = cols[~mask[num_sink:row + 1]]
    if len(others) == 0:
        return True, ""
    worst_chosen = hi[chosen].min()
    best_other = lo[others].max()
    if best_other > worst_chosen:
        c = int(others[np.argmax(lo[others])])
        return False, f"row {row}: column {c} (s={s[c]:.6f}) outranks chosen set {sorted(chosen.tolist())}"
    return True, ""


# ---------------------------------------------------------------------------
# The reference's approximate top-8 (WarpSelect<2, 8, 16>, patch:477-723)
# ---------------------------------------------------------------------------

LANE_QUEUE = 6      # LocalK: packed candidates one lane keeps (patch:501)
ROW_LANES = 4       # LogicalWarp: lanes that share one accumulator row (patch:502)


def warpselect_lane(col):
    """Lane (of the four row-mates) that holds column ``col`` of the QK
    accumulator: an SM90 wgmma C fragment gives lane l of a quad the column
    pairs 8j + 2l, 8j + 2l + 1 of its rows (the coordinates ``update_row``
    reads through tScS_selector, patch:282-286, 586-589).  Tiles start at
    multiples of kBlockN (a multiple of 8), so the class is a function of the
    absolute column."""
    return (np.asarray(col, dtype=np.int64) % 8) // 2


def warpselect_topk(raw_scores, *, row, num_sink, kappa=8, tile=128):
    """The reference's approximate top-8 of one query row, restated.

    Each lane keeps the ``LANE_QUEUE`` largest packed keys (quantised score <<
    17 | column) among the eligible columns of its class (``insert`` keeps a
    sorted queue and admits a candidate only above its last entry,
    patch:556-596), and ``write_row`` merges the four sorted queues by
    repeatedly taking the largest head (patch:640-690), i.e. the top 8 of
    their union.  The tile skip (a tile is passed over when every lane's own
    tile max is at most its sixth key's score, patch:578-583) is applied per
    lane over tiles of ``tile`` columns in the kernel's order, the diagonal tile
    first and then backwards; it can only pass over a candidate whose key equals
    the lane's sixth key, and every such candidate has a smaller column than
    the resident key (it comes from a later-processed, lower tile), so it would
    not have been admitted either: the result equals the per-lane top-6
    without the skip.  Both are computed and the equality asserted.  Masked
    columns (beyond the row) never reach the output for rows with at least
    kappa eligible columns, so they are left out.

    ``raw_scores`` holds the scores of columns 0..row (float64 or float32;
    quantised in float32).  Returns the 8 chosen columns in the merge's
    output order (descending packed key)."""
    if kappa != 8:
        raise ValueError("the reference's WarpSelect is specialised for kappa = 8 only")
    s = np.asarray(raw_scores)[:row + 1].astype(np.float32)
    cols = np.arange(num_sink, row + 1)
    packed = pack_candidates(quantise_score(s[num_sink:row + 1]), cols)
    lanes = warpselect_lane(cols)
    queues = []
    for lane in range(ROW_LANES):
        own = np.sort(packed[lanes == lane])[::-1][:LANE_QUEUE]
        queues.append(own)
    # the streaming form with the tile skip, lane by lane
    for lane in range(ROW_LANES):
        q = []                                  # sorted descending, at most LANE_QUEUE
        last_tile = row // tile
        for t in range(last_tile, -1, -1):
            lo, hi = t * tile, min(row, t * tile + tile - 1)
            sel = (cols >= lo) & (cols <= hi) & (lanes == lane)
            if not sel.any():
                continue
            tile_keys = packed[sel]
            tile_max = s[cols[sel]].max()
            if len(q) == LANE_QUEUE and tile_max <= dequantise_key(q[-1] >> INDEX_BITS):
                continue
            for cand in tile_keys:              # ascending columns inside the tile
                if len(q) < LANE_QUEUE or cand > q[-1]:
                    q.append(int(cand))
                    q.sort(reverse=True)
                    del q[LANE_QUEUE:]
        assert q == queues[lane].tolist(), "the tile skip changed a lane queue"
    merged = np.sort(np.concatenate(queues))[::-1][:kappa]
    return (merged & ((1 << INDEX_BITS) - 1)).astype(np.int64)


__all__ = ["consistent_topk", "dequantise_key", "pack_candidates", "prefill_attention_topk", "prefill_rows",
           "quantise_score", "row_scores", "topk_row_skip", "warpselect_lane", "warpselect_topk"]
