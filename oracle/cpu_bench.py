"""Multi-process CPU baseline runner (MEASUREMENT INFRASTRUCTURE ONLY).

Only ``bench.py``'s ``cpu_baseline`` legs start this module, as plain child
processes (``python -m oracle.cpu_bench <kind> <inputs.npz> <seconds> <worker>
<workers>``) that import numpy and the oracle only, so they never touch the
GPU.  Each worker runs the numpy oracle on the host cores, single-threaded,
and prints one JSON line; bench.py adds the workers' work up.

kinds:
  decode     decode layer-steps of one layer state (ckv_oracle.decode_step)
  prefill    random (row, head) pairs of a prefill (prefill.prefill_rows)
  state      the state build of the graphs g with g % workers == worker
  partition  Leiden + relabel of the graphs g with g % workers == worker
"""

from __future__ import annotations

import json
import sys
import time

import numpy as np


def _decode(z, seconds, worker):
    from oracle import ckv_oracle as co

    deltas = co.DeltaChunks(*(z[f"d{i}"] for i in range(11)))
    st = co.LayerState(
        centroids=z["centroids"], community_sizes=z["community_sizes"], community_counts=z["community_counts"],
        community_weight=z["community_weight"], total_weight=z["total_weight"],
        token_communities=z["token_communities"], deltas=deltas, to_graph=z["to_graph"], to_kv=z["to_kv"],
        member_offsets=z["member_offsets"], member_positions=z["member_positions"],
        current_position=z["current_position"], fp8=True)
    p = z["params"]
    params = co.StepParams(group_size=int(p[0]), num_sink=int(p[1]), token_budget=int(p[2]), local_window=int(p[3]))
    q, k, v = z["q"], z["k"], z["v"]
    max_steps = int(p[4])
    steps, t0 = 0, time.perf_counter()
    while True:
        co.decode_step(st, q, k, v, params)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds or steps >= max_steps:
            break
    return {"steps": steps, "seconds": el}


def _prefill(z, seconds, worker):
    from oracle import prefill as op

    q, k, v = z["q"], z["k"], z["v"]
    scale, sinks, kappa = float(z["params"][0]), int(z["params"][1]), int(z["params"][2])
    S, Hq = q.shape[0], q.shape[1]
    rng = np.random.default_rng(1000 + worker)
    cols, n, t0 = 0, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds and n < 4096:
        r = int(rng.integers(0, S))
        h = int(rng.integers(0, Hq))
        op.prefill_rows(q, k, v, [r], [h], softmax_scale=scale, num_sink=sinks, kappa=kappa)
        cols += r + 1
        n += 1
    return {"rows": n, "cols": cols, "seconds": time.perf_counter() - t0}


def _state(z, seconds, worker, workers):
    from oracle import ckv_oracle as co

    ids, kn, ti, ts, pos = z["ids"], z["keys"], z["tk_idx"], z["tk_sc"], z["pos"]
    sinks, max_decode, seq, cap = (int(x) for x in z["params"][:4])
    lam = float(z["lam"][0])
    mine = [g for g in range(ids.shape[0]) if g % workers == worker]
    t0 = time.perf_counter()
    for g in mine:
        sl = slice(g, g + 1)
        counts = (ids[sl, sinks:].max(axis=1) + 1).astype(np.int32)
        mp = np.zeros(1, np.int32)
        co.build_member_csr(ids[sl], counts, num_sink=sinks)
        co.compute_centroids(ids[sl], counts, kn[sl], to_graph=mp, to_kv=mp, num_sink=sinks,
                             max_decode_tokens=max_decode)
        sn, dn, wn = co.build_adjacency(ti[sl], ts[sl], pos[sl], seq_len=seq, lam=lam)
        co.init_modularity_state(ids[sl], sn, dn, wn, community_capacity=cap, seq_len=seq)
    return {"graphs": len(mine), "seconds": time.perf_counter() - t0}


def _partition(z, seconds, worker, workers):
    from oracle import leiden as L

    src, dst, w = z["src"], z["dst"], z["w"]
    seq, graphs, iters = (int(x) for x in z["params"][:3])
    mine = [g for g in range(graphs) if g % workers == worker]
    t0 = time.perf_counter()
    for g in mine:
        one = (src // seq) == g
        L.partition_labels(src[one] - g * seq, dst[one] - g * seq, w[one], graphs=1, seq_len=seq, resolution=1.0,
                           max_inner_iter=iters, seed=0)
    return {"graphs": len(mine), "seconds": time.perf_counter() - t0}


def main(argv):
    kind, path, seconds, worker, workers = argv[1], argv[2], float(argv[3]), int(argv[4]), int(argv[5])
    z = dict(np.load(path, allow_pickle=False))
    if kind == "decode":
        out = _decode(z, seconds, worker)
    elif kind == "prefill":
        out = _prefill(z, seconds, worker)
    elif kind == "state":
        out = _state(z, seconds, worker, workers)
    elif kind == "partition":
        out = _partition(z, seconds, worker, workers)
    else:
        raise SystemExit(f"unknown kind {kind}")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main(sys.argv)
