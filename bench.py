"""Sparse-decode benchmark on one MI355X (stacked to a
36-layer Qwen3-8B attention stack).

A step is one decode token through 36 independent Qwen3-8B-shaped attention
layers (32 query / 8 KV heads, head_dim 128, bf16 KV, 32,768-token context,
QUERY_GROUP graphs with 512 Zipf(1.1) communities per KV head, 2,048-token
budget + 128-token recent window, 10 sinks, modularity-gain online update).
Each layer owns its own KV cache and graph state (4.8 GB in total).  A step is
captured in a HIP graph (each layer's online update rides in the next layer's
launch, the last layer's in the next step's first launch); four such graphs
whose layers read different queries are replayed in rotation, so a layer's
gathered rows recur only after more than 1 GB of other traffic (the Infinity
Cache holds 256 MB).  Inputs are resident in HBM before timing starts.

Prints one JSON line: the benchmark contract's fields (value = tokens/s over
the K timed steps), the median and 10th/90th percentile of the per-step event
times, `roofline` (the step's dominant kernel, the cooperative selection +
attention + merge launch: algorithmic bytes per launch over its graph-timed
duration; `traffic` from the committed rocprofv3 counter summary when
present) and `cpu_baseline` (the numpy oracle on copies of one layer, one
process per host core).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from community_kv_amd import _native as nat  # noqa: E402
from community_kv_amd.attention.kernels import _abi  # noqa: E402
from community_kv_amd.config import CommunityKVConfig, GraphAggregation  # noqa: E402
from community_kv_amd.graph.partition import build_layer_from_labels  # noqa: E402
from community_kv_amd.runtime import DecodeRuntime  # noqa: E402

HBM_PEAK_GBS = 8000.0
LAYERS = 36
HQ, HKV, D = 32, 8, 128
SEQ = 32768
COMMUNITIES = 512
BUDGET = 2048
WINDOW = 128
SINKS = 10


def zipf_labels(rng, seq, sinks, communities):
    n = seq - sinks
    raw = np.clip(rng.zipf(1.1, size=communities).astype(np.float64), 8, 1024)
    sizes = np.maximum(1, np.round(raw * (n / raw.sum()))).astype(np.int64)
    diff = n - int(sizes.sum())
    order = np.argsort(-sizes, kind="stable")
    i = 0
    while diff:
        j = order[i % communities]
        step = 1 if diff > 0 else -1
        if sizes[j] + step >= 1:
            sizes[j] += step
            diff -= step
        i += 1
    lab = np.repeat(np.arange(communities, dtype=np.int32), sizes)
    rng.shuffle(lab)
    out = np.zeros(seq, np.int32)
    out[sinks:] = lab
    return out


PREFILL_SEQ = 32768
PREFILL_CLUSTERS = 256
PREFILL_KAPPA = 16


def planted_prefill_inputs(device, seq=PREFILL_SEQ, hq=HQ, hkv=HKV, clusters=PREFILL_CLUSTERS, cosine=0.6,
                           block=128, seed=0):
    """BASELINE config 5 inputs: q/k/v [1, seq, heads, 128] bf16.  Each
    ``block``-token block belongs to one of ``clusters`` clusters; a q/k row is
    sqrt(cosine) * center + sqrt(1 - cosine) * noise with center and noise
    ~N(0, 1/128) (unit expected norm), so two rows of one cluster have cosine
    ~``cosine``.  Values ~N(0, 1/128)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    blocks = -(-seq // block)
    lab = torch.randint(0, clusters, (blocks,), device=device, generator=gen).repeat_interleave(block)[:seq]
    scale = D ** -0.5
    centers = torch.randn(hkv, clusters, D, device=device, generator=gen) * scale
    a, b = cosine ** 0.5, (1 - cosine) ** 0.5

    def rows(heads, group):
        x = torch.empty(1, seq, heads, D, device=device, dtype=torch.bfloat16)
        for h in range(heads):
            noise = torch.randn(seq, D, device=device, generator=gen) * scale
            x[0, :, h] = (a * centers[h // group, lab] + b * noise).to(torch.bfloat16)
        return x

    k = rows(hkv, 1)
    q = rows(hq, hq // hkv)  # a query row shares its KV head's cluster centers
    v = (torch.randn(1, seq, hkv, D, device=device, generator=gen) * scale).to(torch.bfloat16)
    return q, k, v


QUERY_SETS = 4  # query variants per layer, replayed in rotation by the timed step


def build_stack(device, layers, max_decode, seed=0, seq_lens=None, communities=None, budget=BUDGET, window=WINDOW,
                query_sets=1, aggregation=GraphAggregation.QUERY_GROUP):
    """`layers` independent layer states (config 2 by default).  With
    `seq_lens` / `communities` (one entry per layer) the entries are the
    sequences of a ragged batch instead (config 4).  Each entry carries
    `query_sets` decode calls that share the layer's state and workspace but
    read different queries (each near another random community centre).
    PER_QUERY_HEAD: every query head gets its own graph, labelled like its
    KV head's keys."""
    cfg = CommunityKVConfig(token_budget=budget, num_sink=SINKS, lam=0.5, aggregation=aggregation,
                            local_window=window)
    runtime = DecodeRuntime(cfg)
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device).manual_seed(seed)
    stack = []
    for li in range(layers):
        seq = SEQ if seq_lens is None else int(seq_lens[li])
        comms = COMMUNITIES if communities is None else int(communities[li])
        cap = seq + max_decode + 1
        labels = torch.from_numpy(np.stack([zipf_labels(rng, seq, SINKS, comms) for _ in range(HKV)])).to(device)
        centers = torch.randn(HKV, comms, D, device=device, generator=gen)
        key = torch.empty(HKV, cap, D, device=device, dtype=torch.bfloat16)
        for h in range(HKV):
            noise = torch.randn(seq, D, device=device, generator=gen)
            key[h, :seq] = (centers[h, labels[h].long()] + 0.3 * noise).to(torch.bfloat16)
            extra = torch.randint(0, comms, (cap - seq,), device=device, generator=gen)
            key[h, seq:] = (centers[h, extra] + 0.3 * torch.randn(cap - seq, D, device=device, generator=gen)).to(
                torch.bfloat16)
        value = torch.randn(HKV, cap, D, device=device, generator=gen).to(torch.bfloat16)
        ids = labels.repeat_interleave(HQ // HKV, 0) if aggregation == GraphAggregation.PER_QUERY_HEAD else labels
        part = build_layer_from_labels(layer_idx=li, community_ids=ids, keys=key[:, :seq], num_sink=SINKS,
                                       max_decode_tokens=max_decode, query_heads=HQ, aggregation=aggregation)
        part.community_weight.uniform_(0.5, 2.0, generator=gen)
        part.total_weight.fill_(float(part.community_weight[0].sum()))
        layer = runtime.prepare_partitioned_layer(part)
        conv = layer.converted
        queries, calls = [], []
        for _ in range(query_sets):
            pick = torch.randint(0, comms, (HKV,), device=device, generator=gen)
            query = (centers[torch.arange(HKV, device=device), pick].repeat_interleave(HQ // HKV, 0)
                     + 0.5 * torch.randn(HQ, D, device=device, generator=gen)).to(torch.bfloat16).contiguous()
            queries.append(query)
            calls.append(layer.workspace.call(query=query, key=key, value=value, csr=conv.csr, state=conv.mutable,
                                              sink_positions=layer.sink_positions,
                                              current_position=conv.current_position, softmax_scale=D ** -0.5,
                                              lam=cfg.lam))
        stack.append(dict(layer=layer, query=queries[0], key=key, value=value, call=calls[0], calls=calls, seq=seq))
    return runtime, stack


def capture(fn, device):
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    torch.cuda.synchronize(device)
    return graph


def time_graph(graph, reps, device):
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(device)
    start.record()
    for _ in range(reps):
        graph.replay()
    stop.record()
    torch.cuda.synchronize(device)
    return start.elapsed_time(stop) / reps  # ms


def time_rotation(graphs, steps, device):
    """Replays graphs[i % len(graphs)] for i < steps between two device
    synchronisations; returns (mean ms per step over the whole timed region,
    per-step ms from events around each replay)."""
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    stops = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize(device)
    for i in range(steps):
        starts[i].record()
        graphs[i % len(graphs)].replay()
        stops[i].record()
    torch.cuda.synchronize(device)
    per = [a.elapsed_time(b) for a, b in zip(starts, stops)]
    return starts[0].elapsed_time(stops[-1]) / steps, per


def algorithmic_bytes(stack):
    """Per-layer bytes: attention (K+V rows of valid slots, slot indices, q),
    whole step (+ centroid table, sizes, scores, update) and the centroid
    table (+ sizes, scores) alone."""
    att, step, cent = [], [], []
    for entry in stack:
        sel = entry["layer"].workspace.selection
        slots = sel.slot_positions
        valid = int((slots >= 0).sum().item())
        q_bytes = HQ * D * 2
        a = valid * 2 * D * 2 + slots.numel() * 4 + q_bytes
        counts = entry["layer"].converted.mutable.community_counts
        c_bytes = int(counts.sum().item()) * (D * 1 + 4 + 2)
        s = a + c_bytes + HQ * D * 2 + (D * 2 + 256) * HKV
        att.append(a)
        step.append(s)
        cent.append(c_bytes)
    tokens = float(np.mean([int((e["layer"].workspace.selection.slot_positions >= 0).sum()) / HKV for e in stack]))
    return float(np.mean(att)), float(np.mean(step)), tokens, float(np.mean(cent))


def profiled_traffic(key="traffic_bytes_per_launch"):
    """HBM bytes per fused selection + attention launch from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a plain copy of
    known size): `key` names the launch (bare, or carrying the previous layer's
    update), None when the summary or the line is absent."""
    path = os.path.join(ROOT, "profiles", "select_attend_config2_traffic.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1])
    return None


def cpu_workers():
    """Host cores the CPU baselines use: every core this process may use.  On
    a machine that sets OMP_NUM_THREADS to the job's CPU share (the one-GPU box
    sets 16 and counts worker processes against it, while os.cpu_count()
    reports the whole host), that share; otherwise os.cpu_count()."""
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    total = os.cpu_count() or 1
    return max(1, min(share, total) if share > 0 else total)


def cpu_core_note(workers):
    """How the core count was chosen, for cpu_baseline.sample."""
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    if share > 0 and workers == min(share, os.cpu_count() or 1):
        return (f"{workers} worker processes = this job's CPU share (OMP_NUM_THREADS={share}; "
                f"os.cpu_count() reports {os.cpu_count()} host-wide)")
    return f"{workers} worker processes = os.cpu_count()"


def run_cpu_workers(kind, arrays, seconds):
    """Runs `kind` of oracle/cpu_bench.py in cpu_workers() single-threaded child
    processes (numpy + the oracle only; they never touch the GPU) on the
    arrays saved to a temporary .npz; returns (per-worker results, workers,
    wall seconds)."""
    import subprocess
    import tempfile

    workers = cpu_workers()
    env = dict(os.environ, OMP_NUM_THREADS="1", OPENBLAS_NUM_THREADS="1", MKL_NUM_THREADS="1",
               PYTHONPATH=ROOT + os.pathsep + os.environ.get("PYTHONPATH", ""))
    with tempfile.TemporaryDirectory(prefix="ckv_cpu_") as tmp:
        path = os.path.join(tmp, "inputs.npz")
        np.savez(path, **arrays)
        t0 = time.perf_counter()
        procs = [subprocess.Popen([sys.executable, "-m", "oracle.cpu_bench", kind, path, str(seconds), str(i),
                                   str(workers)], stdout=subprocess.PIPE, stderr=subprocess.PIPE, env=env, cwd=ROOT)
                 for i in range(workers)]
        outs = []
        for pr in procs:
            out, err = pr.communicate(timeout=seconds * 4 + 300)
            if pr.returncode != 0:
                raise RuntimeError(f"cpu baseline worker failed: {err.decode()[-2000:]}")
            outs.append(json.loads(out.decode().strip().splitlines()[-1]))
        wall = time.perf_counter() - t0
    return outs, workers, wall


def cpu_baseline(entry, seconds=20.0):
    """Oracle decode layer-steps (numpy restatement of the reference semantics)
    on copies of one layer's state, one per host core, for a bounded time."""
    layer = entry["layer"]
    conv = layer.converted
    m = conv.mutable
    npy = lambda t: t.detach().cpu().numpy().copy()
    arrays = dict(centroids=npy(m.centroids.view(torch.uint8)), community_sizes=npy(m.community_sizes),
                  community_counts=npy(m.community_counts), community_weight=npy(m.community_weight),
                  total_weight=npy(m.total_weight), token_communities=npy(m.token_communities),
                  to_graph=npy(m.retrieval_to_graph), to_kv=npy(m.retrieval_to_kv),
                  member_offsets=npy(conv.csr.member_offsets), member_positions=npy(conv.csr.member_positions),
                  current_position=npy(conv.current_position),
                  q=entry["query"].float().cpu().numpy(), k=entry["key"].float().cpu().numpy(),
                  v=entry["value"].float().cpu().numpy(),
                  params=np.array([HQ // HKV, SINKS, BUDGET, WINDOW, 50], np.int64))
    for i, t in enumerate(m.deltas.tensors()):
        arrays[f"d{i}"] = npy(t)
    outs, workers, wall = run_cpu_workers("decode", arrays, seconds)
    steps = sum(o["steps"] for o in outs)
    rate = sum(o["steps"] / o["seconds"] for o in outs)  # layer-steps per second over all cores
    return {"value": rate / LAYERS, "unit": "tokens/s", "cores": workers, "kind": "port",
            "sample": f"{steps} decode layer-steps of one config-2 layer through the numpy oracle on {workers} "
                      f"host cores ({workers / rate * 1e3:.1f} ms per layer-step per core), scaled to 36 layers; "
                      f"{cpu_core_note(workers)}"}


MFMA_BF16_PEAK_TFLOPS = 2500.0


def prefill_cpu_baseline(q, k, v, scale, sinks, kappa, seconds):
    """Oracle prefill rows (numpy) at random positions of the same inputs, one
    worker per host core, scaled to the whole prefill by each row's causal
    length."""
    arrays = dict(q=q[0].float().cpu().numpy(), k=k[0].float().cpu().numpy(), v=v[0].float().cpu().numpy(),
                  params=np.array([scale, sinks, kappa], np.float64))
    outs, workers, wall = run_cpu_workers("prefill", arrays, seconds)
    S, Hq = q.shape[1], q.shape[2]
    cols_per_s = sum(o["cols"] / o["seconds"] for o in outs)
    rows = sum(o["rows"] for o in outs)
    total_cols = Hq * S * (S + 1) / 2
    return {"value": cols_per_s / total_cols, "unit": "prefills/s", "cores": workers, "kind": "port",
            "sample": f"{rows} random (row, head) pairs of the config-5 prefill through the numpy oracle on "
                      f"{workers} host cores, scaled by causal columns to the whole prefill"}


def run_prefill(args, device, emit=True):
    from community_kv_amd.attention.flash_attention import prefill_attention_topk

    q, k, v = planted_prefill_inputs(device, seq=args.prefill_seq)
    S = q.shape[1]
    scale = D ** -0.5
    run = lambda: prefill_attention_topk(q, k, v, softmax_scale=scale, num_sink=SINKS, kappa=PREFILL_KAPPA)
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize(device)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        run()
    stop.record()
    torch.cuda.synchronize(device)
    ms = start.elapsed_time(stop) / args.steps
    flops = 4.0 * D * HQ * S * (S + 1) / 2  # causal QK^T + PV
    tflops = flops / (ms * 1e-3) / 1e12
    result = {
        "metric": "prefill_edge_export_ms_32k_qwen3_8b_layer",
        "value": ms,
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (planted 256-cluster q/k blocks, cosine 0.6; N(0,1/128) values)",
        "config": {"workload": "BASELINE config 5: causal prefill, 32/8 heads, head_dim 128, top-16 edges per row",
                   "seq_len": S, "query_heads": HQ, "kv_heads": HKV, "kappa": PREFILL_KAPPA, "num_sink": SINKS},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": tflops / MFMA_BF16_PEAK_TFLOPS, "traffic": None,
                     "kernel": "prefill_mfma_kernel<16>", "flops_per_launch": flops},
    }
    if not emit:
        return result
    if not args.no_cpu:
        result["cpu_baseline"] = prefill_cpu_baseline(q, k, v, scale, SINKS, PREFILL_KAPPA, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return result


STATE_KAPPA = 8  # the prefill edge width the runtime requests


def run_state(args, device):
    """GPU state assembly of one config-2 layer from labels and the prefill's
    top-k edges (the first 'next' row after the decode path): 8 QUERY_GROUP
    graphs x 32,768 positions, 512 Zipf(1.1) communities, bf16 keys, top-8
    edges of every row of all 32 query heads.  Times ckv_build_layer_state
    (CSR, centroids, sizes, modularity weights, token table) with inputs and
    outputs resident; the label-count read-back that sizes the outputs is
    set-up."""
    from community_kv_amd.graph.kernels.state_build import StateBuild, TopkEdges

    rng = np.random.default_rng(3)
    gen = torch.Generator(device=device).manual_seed(3)
    labels = torch.from_numpy(np.stack([zipf_labels(rng, SEQ, SINKS, COMMUNITIES) for _ in range(HKV)])).to(device)
    keys = torch.randn(HKV, SEQ + 64, D, device=device, generator=gen).to(torch.bfloat16)[:, :SEQ]
    row0 = SINKS + STATE_KAPPA - 1
    rows = SEQ - row0
    tk_idx = torch.randint(SINKS, SEQ, (HQ, rows, STATE_KAPPA), device=device, generator=gen, dtype=torch.int32)
    tk_sc = torch.rand(HQ, rows, STATE_KAPPA, device=device, generator=gen)
    maps = torch.arange(HKV, dtype=torch.int32, device=device)
    max_decode = 64
    lam = 0.5
    build = StateBuild(labels, keys, retrieval_to_graph=maps, retrieval_to_kv=maps, num_sink=SINKS,
                       max_decode_tokens=max_decode,
                       topk_edges=TopkEdges(indices=tk_idx, scores=tk_sc, row0=row0, group=HQ // HKV, lam=lam))
    for _ in range(args.warmup):
        build.run()
    torch.cuda.synchronize(device)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        build.run()
    stop.record()
    torch.cuda.synchronize(device)
    ms = start.elapsed_time(stop) / args.steps
    out = build.out
    cap = out.community_sizes.shape[1]
    nsink = SEQ - SINKS
    entries = HQ * rows * STATE_KAPPA
    algorithmic = (HKV * SEQ * 4                      # labels
                   + HKV * nsink * D * 2              # keys, each non-sink row once
                   + entries * (4 + 4)                # top-k indices and scores
                   + entries * 4 + HQ * rows * 4      # the column and row labels
                   + HKV * nsink * 4                  # member positions
                   + out.member_offsets.numel() * 4
                   + HKV * cap * (D + 4)              # centroids (e4m3) + sizes
                   + out.token_communities.numel() * 4
                   + HKV * (cap + 1) * 4)             # modularity weights
    gbs = algorithmic / (ms * 1e-3) / 1e9
    result = {
        "metric": "state_build_us_32k_qwen3_8b_layer",
        "value": ms * 1e3,
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32+bf16->e4m3",
        "data": "synthetic (Zipf(1.1) labels, N(0,1) bf16 keys, uniform random top-8 columns and scores)",
        "config": {"workload": "GPU state assembly from labels and prefill top-8 edges, config-2 layer (8 graphs "
                               "x 32768, 512 communities, 32 query heads)", "graphs": HKV, "seq_len": SEQ,
                   "communities": COMMUNITIES, "kappa": STATE_KAPPA, "lam": lam},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "ckv_build_layer_state (8 launches, whole build)", "bytes_per_launch": algorithmic},
    }
    if not args.no_cpu:
        group = HQ // HKV
        pos = np.tile(np.arange(row0, row0 + rows), group)[None].repeat(HKV, 0)
        arrays = dict(ids=labels.cpu().numpy(), keys=keys.float().cpu().numpy(),
                      tk_idx=tk_idx.cpu().numpy().reshape(HKV, group * rows, STATE_KAPPA),
                      tk_sc=tk_sc.cpu().numpy().reshape(HKV, group * rows, STATE_KAPPA), pos=pos,
                      params=np.array([SINKS, max_decode, SEQ, cap], np.int64), lam=np.array([lam], np.float64))
        outs, workers, wall = run_cpu_workers("state", arrays, 0.0)
        result["cpu_baseline"] = {"value": wall * 1e6, "unit": "us", "cores": workers, "kind": "port",
                                  "sample": f"the whole layer build (numpy oracle: CSR, centroids, coalesced adjacency, "
                                            f"modularity weights), graphs split over {workers} host cores, wall time "
                                            f"including worker start-up"}
    print(json.dumps(result), flush=True)


def run_partition(args, device):
    """Prefill partition of one config-2 layer (the second 'next' row): the
    top-8 edges of all 32 query heads from the prefill kernel on planted
    config-5 style inputs (32,768 tokens, 256 clusters), grouped into 8
    QUERY_GROUP graphs, then ``partition_graphs``: build_adjacency (device
    torch ops), native multi-level Leiden (ckv_batched_leiden /
    ckv_aggregate_coo / ckv_densify_*), isolated fill and dense remap.  The
    timed region is the whole partition; the Leiden part is timed alone too."""
    from community_kv_amd.attention.flash_attention import prefill_attention_topk
    from community_kv_amd.graph import partition as P
    from community_kv_amd.graph.leiden import run_leiden

    q, k, v = planted_prefill_inputs(device, seq=args.prefill_seq)
    S = q.shape[1]
    out = prefill_attention_topk(q, k, v, softmax_scale=D ** -0.5, num_sink=SINKS, kappa=STATE_KAPPA)
    idx, val = out[5][0].contiguous(), out[4][0].contiguous()
    del q, k, v, out
    kw = dict(aggregation="query_group", num_kv_heads=HKV, prefill_seq_len=S, num_sink=SINKS, lam=0.5,
              leiden_resolution=1.0, leiden_seed=0)
    run = lambda: P.partition_graphs(idx, val, **kw)
    g_idx, g_val, pos = P._reshape_by_aggregation(idx, val, aggregation="query_group", num_kv_heads=HKV,
                                                  num_sink=SINKS)
    src, dst, w = P.build_adjacency(g_idx, g_val, pos, seq_len=S, lam=0.5)
    iters = P.leiden_max_iterations(S)
    leiden = lambda: run_leiden(src, dst, w, G=HKV, seq_len=S, max_inner_iter=iters, seed=0)
    for _ in range(args.warmup):
        res = run()
    torch.cuda.synchronize(device)

    def timed(fn):
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize(device)
        return (time.perf_counter() - t0) / args.steps * 1e3

    ms = timed(run)
    leiden_ms = timed(leiden)
    counts = res.community_counts.cpu().tolist()
    result = {
        "metric": "partition_ms_32k_qwen3_8b_layer",
        "value": ms,
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32+f32 (f64 gains)",
        "data": "synthetic (prefill top-8 edges of planted config-5 style q/k/v, 256 clusters, cosine 0.6)",
        "config": {"workload": "prefill partition of a config-2 layer: 8 QUERY_GROUP graphs x 32768 tokens, "
                               "top-8 edges of 32 query heads, lam 0.5, resolution 1, "
                               f"{iters} sweeps per phase", "graphs": HKV, "seq_len": S,
                   "edges": int(src.numel()), "communities_per_graph": counts,
                   "modularity": res.modularity, "leiden_only_ms": leiden_ms},
        "roofline": None,
    }
    if not args.no_cpu:
        arrays = dict(src=src.long().cpu().numpy(), dst=dst.long().cpu().numpy(), w=w.cpu().numpy(),
                      params=np.array([S, HKV, iters], np.int64))
        outs, workers, wall = run_cpu_workers("partition", arrays, 0.0)
        result["cpu_baseline"] = {"value": wall * 1e3, "unit": "ms", "cores": workers, "kind": "port",
                                  "sample": f"numpy oracle Leiden + relabel of the 8 graphs, split over {workers} host "
                                            f"cores, wall time including worker start-up"}
    print(json.dumps(result), flush=True)


GEN_LAYERS = 36
GEN_PROMPT = 65536
GEN_STEPS = 128
GEN_COMMUNITIES = 1024


def qwen3_8b_config(layers):
    from transformers import Qwen3Config

    return Qwen3Config(vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_hidden_layers=layers,
                       num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D, max_position_embeddings=131072,
                       rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=False)


def run_generate(args, device, emit=True):
    """random-init Qwen3-8B-architecture model, synthetic
    prompt, greedy decode through CommunityKVRuntime.generate with
    nearest-centroid assignment.  Decode throughput = (steps) / (wall time of a
    prompt+steps generation - wall time of a prompt+1 generation)."""
    from transformers import Qwen3ForCausalLM

    from community_kv_amd import CommunityKVAttention, CommunityKVConfig, CommunityKVRuntime
    from community_kv_amd.config import PartitionConfig

    layers, prompt_len, steps = args.gen_layers, args.gen_prompt, args.gen_steps
    torch.manual_seed(0)
    with torch.device(device):
        model = Qwen3ForCausalLM(qwen3_8b_config(layers))
    model = model.to(torch.bfloat16).eval()
    prompt = torch.randint(0, 151936, (1, prompt_len), generator=torch.Generator().manual_seed(1)).to(device)
    rng = np.random.default_rng(7)
    label_cache = {}

    def labels(layer_idx, keys, topk_indices, topk_scores):
        # seeded per layer and KV head: Zipf(1.1) sizes over ~1024 communities
        if layer_idx not in label_cache:
            label_cache[layer_idx] = torch.from_numpy(np.stack([
                zipf_labels(rng, keys.shape[1], SINKS, GEN_COMMUNITIES) for _ in range(keys.shape[0])]))
        return label_cache[layer_idx].to(keys.device)

    cfg = CommunityKVConfig(token_budget=BUDGET, num_sink=SINKS, aggregation=GraphAggregation.QUERY_GROUP,
                            local_window=WINDOW, assignment="nearest_centroid")
    with CommunityKVRuntime(config=cfg, partition=PartitionConfig(overlap=not args.partition_inline),
                            num_layers=layers, max_decode_tokens=steps,
                            label_provider=None if args.leiden else labels) as runtime:
        CommunityKVAttention(runtime).register()
        model.set_attn_implementation("community_kv")

        def timed(new_tokens):
            torch.cuda.synchronize(device)
            t0 = time.perf_counter()
            with torch.inference_mode():
                out = runtime.generate(model, prompt, max_new_tokens=new_tokens)
            torch.cuda.synchronize(device)
            dt = time.perf_counter() - t0
            print(f"generate: {new_tokens} new tokens after a {prompt_len}-token prompt in {dt:.2f} s",
                  file=sys.stderr, flush=True)
            return dt, out

        # every generation repeats the prefill (and its partitions), so one warm-up is enough
        for _ in range(min(max(0, args.warmup), 1)):
            timed(2)
        t_prefill, _ = timed(1)
        t_full, out = timed(steps + 1)
    decode_s = t_full - t_prefill
    tps = steps / decode_s
    result = {
        "metric": "generate_decode_tokens_per_s_qwen3_8b_random_init",
        "value": tps,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": decode_s * 1e3 / steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": ("synthetic (uniform random prompt ids, random-init weights, "
                 + ("communities from the native Leiden on each layer's prefill top-8 edges)" if args.leiden
                    else "Zipf(1.1) labels over ~1024 communities)")),
        "config": {"workload": "BASELINE config 3: random-init Qwen3-8B architecture, greedy decode through "
                               "CommunityKVRuntime.generate, nearest-centroid assignment",
                   "layers": layers, "prompt_tokens": prompt_len, "decode_steps": steps, "token_budget": BUDGET,
                   "local_window": WINDOW, "num_sink": SINKS},
        "prefill_plus_first_token_s": t_prefill,
        "generated_tokens": int(out.shape[-1] - prompt_len),
    }
    if emit:
        print(json.dumps(result), flush=True)
    return result


BATCH = 8
BATCH_MIN, BATCH_MAX = 16384, 131072
BATCH_BUDGET = 4096


def run_batched(args, device, emit=True):
    """a ragged batch of 8 sequences (lengths uniform in
    [16k, 128k], length/64 Zipf communities per KV head, 4096-token budget +
    128 window), one Qwen3-8B-shaped layer; a step decodes one token of every
    sequence with the batched entry point (one selection, attention, merge and
    update launch for all 8 sequences), captured in one HIP graph; `steps` of
    them with online (delta-Q) assignment.  The same step issued sequence by
    sequence is reported beside it."""
    rng = np.random.default_rng(3)
    lens = rng.integers(BATCH_MIN, BATCH_MAX + 1, BATCH)
    comms = [int(n) // 64 for n in lens]
    # every replay appends one token (the deferred pair below: one per layer)
    max_decode = 3 * args.warmup + 3 * args.steps + max(5, args.steps // 4) + 16
    runtime, stack = build_stack(device, BATCH, max_decode, seed=1, seq_lens=lens, communities=comms,
                                 budget=BATCH_BUDGET)
    torch.cuda.synchronize(device)

    from community_kv_amd.attention.kernels._abi import BatchDecode

    batch = BatchDecode([e["call"] for e in stack])
    graph = capture(batch.decode, device)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize(device)
    ms = time_graph(graph, args.steps, device)

    def serial_step():  # the same step issued sequence by sequence (deferred updates)
        pending = None
        for e in stack:
            e["call"].decode_after(pending)
            pending = e["call"]
        pending.update()

    serial_graph = capture(serial_step, device)
    serial_graph.replay()
    serial_ms = time_graph(serial_graph, max(5, args.steps // 4), device)
    # A second layer's batch (the same 8 contexts): the two layers step
    # alternately, each leaving its online update pending to run inside the
    # other's selection launch, as a model's consecutive layers would
    # (ckv_batch_decode_after_update).  Per layer-step = replay / 2.
    _, stack2 = build_stack(device, BATCH, max_decode, seed=2, seq_lens=lens, communities=comms,
                            budget=BATCH_BUDGET)
    batch2 = BatchDecode([e["call"] for e in stack2])

    # The same two layers with every update inline: a layer's K/V rows (137 MB)
    # are no longer still in the 256 MB Infinity Cache when it steps again, as
    # in a model; the single-layer figure above re-reads one layer's rows.
    def inline_pair():
        batch.decode()
        batch2.decode()

    inline_graph = capture(inline_pair, device)
    for _ in range(args.warmup):
        inline_graph.replay()
    inline2_ms = time_graph(inline_graph, args.steps, device) / 2
    del inline_graph
    batch.decode_after(None)
    batch2.decode_after(batch)

    def deferred_pair():
        batch.decode_after(batch2)
        batch2.decode_after(batch)

    deferred_graph = capture(deferred_pair, device)
    for _ in range(args.warmup):
        deferred_graph.replay()
    deferred_ms = time_graph(deferred_graph, args.steps, device) / 2
    batch2.update()
    overflow2 = sum(int(e["layer"].workspace.update.overflow.sum().item()) for e in stack2)
    del deferred_graph

    def attended_bytes(st):
        out = 0
        for e in st:
            slots = e["layer"].workspace.selection.slot_positions
            out += int((slots >= 0).sum().item()) * 2 * D * 2 + slots.numel() * 4 + HQ * D * 2
        return out

    att_bytes = [attended_bytes(stack), attended_bytes(stack2)]
    # ten back-to-back launches per replay, so one replay's fixed cost does not
    # count against the kernel, alternating between the two layers' batches so
    # that no launch finds the previous one's rows in the Infinity Cache (the
    # attention launches write disjoint partials)
    att_graph = capture(lambda: [b.attention_partials() for _ in range(5) for b in (batch, batch2)], device)
    att_graph.replay()
    part_ms = time_graph(att_graph, max(10, args.steps), device) / 10
    achieved = float(np.mean(att_bytes)) / (part_ms * 1e-3) / 1e9
    del att_graph, batch2, stack2
    step_bytes = algorithmic_bytes(stack)[1] * len(stack)
    overflow = sum(int(e["layer"].workspace.update.overflow.sum().item()) for e in stack)
    result = {
        "metric": "batched_ragged_decode_tokens_per_s_qwen3_8b_layer",
        "value": BATCH * 1e3 / ms,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (Gaussian-mixture keys, Zipf(1.1) community sizes, random-init state)",
        "config": {"workload": "BASELINE config 4: batch 8, ragged contexts U[16384, 131072], length/64 communities "
                               "per KV head, budget 4096 + window 128, one Qwen3-8B-shaped layer, delta-Q update",
                   "context_lengths": [int(n) for n in lens], "token_budget": BATCH_BUDGET, "local_window": WINDOW},
        "us_per_batch_step": ms * 1e3,
        "us_per_batch_step_sequence_by_sequence": serial_ms * 1e3,
        "us_per_layer_step_two_layers": inline2_ms * 1e3,
        "us_per_layer_step_deferred_update": deferred_ms * 1e3,
        "two_layer_note": ("us_per_batch_step: one layer's batch stepped repeatedly (its K/V rows partly stay in "
                           "the Infinity Cache); us_per_layer_step_two_layers: two layers' batches of the same "
                           "contexts stepped alternately, every update inline; us_per_layer_step_deferred_update: "
                           "the same two layers, each layer's online update run inside the other layer's selection "
                           "launch (ckv_batch_decode_after_update)"),
        "step_algorithmic_bytes": step_bytes,
        "step_hbm_frac": step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "overflow_flags": overflow + overflow2,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "attend_mfma_batch_kernel (gather + split partials of all 8 sequences)",
                     "bytes_per_launch": float(np.mean(att_bytes)),
                     "note": "ten launches per graph replay alternating between two layers' batches"},
        "attention_partials_kernel_us": part_ms * 1e3,
    }
    if emit:
        print(json.dumps(result), flush=True)
    return result


def side_configs(args, device):
    """Short timed runs of configs 5 (prefill edge export) and 4 (batched
    ragged decode) for the default line, each with its own roofline: a few
    launches / graph replays, so the default command stays short."""
    import types

    out = {}
    pre = run_prefill(types.SimpleNamespace(prefill_seq=PREFILL_SEQ, warmup=3, steps=5, no_cpu=True), device,
                      emit=False)
    out["prefill_ms"] = pre["value"]
    out["prefill_tflops"] = pre["roofline"]["achieved"]
    out["prefill_mfma_frac"] = pre["roofline"]["frac"]
    torch.cuda.empty_cache()
    bat = run_batched(types.SimpleNamespace(warmup=3, steps=20), device, emit=False)
    out["batched_us_per_step"] = bat["us_per_batch_step"]
    out["batched_us_per_layer_step_two_layers"] = bat["us_per_layer_step_two_layers"]
    out["batched_us_per_layer_step_deferred_update"] = bat["us_per_layer_step_deferred_update"]
    out["batched_tokens_per_s"] = bat["value"]
    out["batched_attention_kernel_us"] = bat["attention_partials_kernel_us"]
    out["batched_hbm_frac"] = bat["roofline"]["frac"]
    out["batched_step_hbm_frac"] = bat["step_hbm_frac"]
    torch.cuda.empty_cache()
    gen = run_generate(types.SimpleNamespace(gen_layers=GEN_LAYERS, gen_prompt=GEN_PROMPT, gen_steps=GEN_STEPS,
                                             warmup=10, leiden=False, partition_inline=False, no_cpu=True),
                       device, emit=False)
    out["generate_tokens_per_s"] = gen["value"]
    out["generate_ms_per_token"] = gen["ms_per_step"]
    out["generate_prefill_plus_first_token_s"] = gen["prefill_plus_first_token_s"]
    out["side_configs"] = ("prefill_*: BASELINE config 5 (32,768-token causal prefill, 32/8 heads, top-16 edges), "
                           "mean of 5 launches after 3 warm-up launches (the clock ramps over the first), MFMA roofline = 4*128*32*S(S+1)/2 FLOP / time / "
                           "2.5 PFLOP/s; batched_*: BASELINE config 4 (8 ragged sequences), mean of 20 graph-replayed "
                           "steps after 3, batched_hbm_frac = the batched attention kernel's algorithmic bytes / its "
                           "time / 8 TB/s, batched_step_hbm_frac = the whole step's algorithmic bytes / step time; generate_*: "
                           "BASELINE config 3 (random-init Qwen3-8B, 65,536-token prompt, 128 greedy steps through "
                           "CommunityKVRuntime.generate, the whole step replayed from one HIP graph)")
    return out


def dense_decode_ms(stack, seq, reps, device):
    """This build's dense bf16 decode (ckv_dense_decode) over the first `seq`
    tokens of every layer's cache, one graph replay per step: ms per step."""
    tiles = -(-seq // 64)
    ws = dict(pm=torch.empty(HQ, tiles, device=device), ps=torch.empty(HQ, tiles, device=device),
              pa=torch.empty(HQ, tiles, D, device=device), out=torch.empty(HQ, D, device=device, dtype=torch.bfloat16),
              lse=torch.empty(HQ, device=device))
    kvs = [_abi.kv_struct(e["query"], e["key"], e["value"]) for e in stack]

    def step():
        s = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
        for kv in kvs:
            nat.check(nat.lib().ckv_dense_decode(ctypes.byref(kv), seq, D ** -0.5, ws["pm"].data_ptr(),
                                                 ws["ps"].data_ptr(), ws["pa"].data_ptr(), ws["out"].data_ptr(),
                                                 ws["lse"].data_ptr(), s))

    graph = capture(step, device)
    graph.replay()
    return time_graph(graph, reps, device)


PAPER_SEQ = 131072
PAPER_BUDGET = 4096
PAPER_H100_US_PER_LAYER = 283.0  # paper Table 5, Qwen3-8B: (4.7 + 5.5) ms per step / 36 layers


def run_paper(args, device):
    """The paper's own decode setting (Table 5: 131k context, budget 4096, 10
    sinks, per-query-head graphs, no window) at the Qwen3-8B layer shape, 36
    layers of synthetic state (length/64 Zipf communities per graph), one
    decode step of every layer per replay with the online update deferred into
    the next layer's launch.  The paper's H100 figure (retrieval + sparse
    attention per layer) is printed beside it for context: other hardware and
    other kernels, so it is not `vs_baseline`."""
    layers = args.layers
    max_decode = args.warmup + args.steps + 8
    runtime, stack = build_stack(device, layers, max_decode, seed=2, seq_lens=[PAPER_SEQ] * layers,
                                 communities=[PAPER_SEQ // 64] * layers, budget=PAPER_BUDGET, window=0,
                                 aggregation=GraphAggregation.PER_QUERY_HEAD)
    torch.cuda.synchronize(device)

    def step_carry(pending):
        for e in stack:
            e["call"].decode_after(pending)
            pending = e["call"]
        return pending

    carried = step_carry(None)
    graph = capture(lambda: step_carry(carried), device)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize(device)
    ms, step_ms = time_rotation([graph], args.steps, device)
    stack[-1]["call"].update()
    dense_ms = dense_decode_ms(stack, PAPER_SEQ, max(3, args.steps // 10), device)
    overflow = sum(int(e["layer"].workspace.update.overflow.sum().item()) for e in stack)
    us_layer = ms * 1e3 / len(stack)
    result = {
        "metric": "sparse_decode_us_per_step_layer_paper_setting",
        "value": us_layer,
        "unit": "us/step/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (Gaussian-mixture keys, Zipf(1.1) community sizes, random-init state)",
        "config": {"workload": "paper Table 5 decode setting at the Qwen3-8B layer shape: ctx 131072, budget 4096, "
                               "10 sinks, PER_QUERY_HEAD graphs, no window, 2048 communities per graph, x36 layers, "
                               "delta-Q update", "layers": len(stack), "context": PAPER_SEQ,
                   "token_budget": PAPER_BUDGET, "num_sink": SINKS},
        "us_per_step_layer_median": float(np.median(step_ms)) * 1e3 / len(stack),
        "dense_us_per_step_layer": dense_ms * 1e3 / len(stack),
        "speedup_vs_dense": dense_ms / ms,
        "paper_h100_retrieval_plus_attention_us_per_layer": PAPER_H100_US_PER_LAYER,
        "overflow_flags": overflow,
    }
    print(json.dumps(result), flush=True)



def run_floor(args, device):
    """Latency probes behind the decode step's cost model: the launch floor of
    a graph-replayed kernel (empty kernels of the cooperative launch's shape),
    the dependent-load round trip at three working-set sizes (L2-, Infinity
    Cache- and HBM-resident random cycles), an agent-scope atomic round trip
    and a workgroup-to-workgroup hand-off.  One JSON line; the model that
    adds them up is written out in the design notes."""
    import ctypes

    from community_kv_amd import _native as nat

    lib = nat.lib()
    out = torch.zeros(2, dtype=torch.int64, device=device)
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)

    def empty_us(blocks, threads, lds, n=36):
        def body():
            for _ in range(n):
                nat.check(lib.ckv_latency_probe(0, None, 0, 0, blocks, threads, lds, None, stream()))
        g = capture(body, device)
        g.replay()
        torch.cuda.synchronize(device)
        return time_graph(g, 50, device) * 1e3 / n

    clock = {}

    def ticks(kind, buf, nbytes, hops):
        """ns per hop from the host's event timing of the one-thread kernel
        (hops long enough that the launch is noise), and the device wall
        clock's tick rate from the same run."""
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        nat.check(lib.ckv_latency_probe(kind, ctypes.c_void_p(buf.data_ptr()), nbytes, hops, 0, 0, 0,
                                        ctypes.c_void_p(out.data_ptr()), stream()))
        t1.record()
        torch.cuda.synchronize(device)
        ms = t0.elapsed_time(t1)
        clock.setdefault("mhz", []).append(int(out[0].item()) / (ms * 1e3))
        return ms * 1e6 / hops

    def chase_ns(nbytes, agent, hops=4000):
        stride = 256  # uint32 entries (1 KiB) between nodes: every hop a new line
        nodes = max(2, nbytes // (4 * stride))
        buf = torch.zeros(nodes * stride, dtype=torch.int32, device=device)
        order = torch.cat([torch.zeros(1, dtype=torch.int64, device=device),
                           1 + torch.randperm(nodes - 1, device=device, dtype=torch.int64)])  # node 0 first
        idx = order * stride
        buf[idx] = torch.roll(idx, -1).to(torch.int32)  # one cycle through every node
        ticks(2 if agent else 1, buf, nbytes, 200)  # warm-up pass
        return ticks(2 if agent else 1, buf, nbytes, hops)

    word = torch.zeros(64, dtype=torch.int32, device=device)
    res = {"metric": "decode_latency_floor_components", "unit": "ns (us where named)", "n_gpus": 1,
           "data": "synthetic probes", "config": {"workload": "latency probes for the decode-step cost model"}}
    res["empty_launch_us_1x64"] = empty_us(1, 64, 0)
    res["empty_launch_us_144x512"] = empty_us(144, 512, 0)
    res["empty_launch_us_144x512_lds130k"] = empty_us(144, 512, 130 * 1024)
    for name, nbytes in (("l2_1MiB", 1 << 20), ("mall_64MiB", 64 << 20), ("hbm_4GiB", 4 << 30)):
        res[f"chase_plain_ns_{name}"] = chase_ns(nbytes, False)
        res[f"chase_agent_ns_{name}"] = chase_ns(nbytes, True)
    res["atomic_agent_rtt_ns"] = ticks(3, word, 256, 4000)
    word.zero_()
    res["handoff_agent_ns"] = ticks(4, word, 256, 2000)
    res["wall_clock_mhz_implied"] = float(np.median(clock["mhz"]))
    # placement of the cooperative decode grid's workgroups on the XCDs
    # (head h's parts are blocks h, h + 8, ...: they share an XCD when block b
    # runs on XCD b % 8)
    blocks = 144
    xcc = torch.zeros(blocks, dtype=torch.int32, device=device)
    for _ in range(20):
        nat.check(lib.ckv_latency_probe(5, ctypes.c_void_p(xcc.data_ptr()), blocks * 4, 0, blocks, 512, 130 * 1024,
                                        None, stream()))
        torch.cuda.synchronize(device)
        ids = xcc.cpu().numpy()
        res.setdefault("xcd_block_mod8_runs", 0)
        res["xcd_block_mod8_runs"] += int(all(ids[b] == ids[b % 8] for b in range(blocks)))
    res["xcd_ids_first_16_blocks"] = [int(x) for x in ids[:16]]
    res["xcd_probe_runs"] = 20
    # practical streaming bandwidth of this GPU, for scale: torch's own copy
    # (read + write) and sum (read) kernels over buffers below and above the
    # 256 MB Infinity Cache, HIP events around 10 launches after 3
    for mib in (256, 4096):
        a = torch.ones((mib << 20) // 4, dtype=torch.float32, device=device)
        b = torch.empty_like(a)
        for name, fn, moved in (("copy", lambda: b.copy_(a), 2), ("sum", lambda: a.sum(), 1)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize(device)
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record()
            for _ in range(10):
                fn()
            t1.record()
            torch.cuda.synchronize(device)
            res[f"torch_{name}_{mib}MiB_TBps"] = moved * (mib << 20) / (t0.elapsed_time(t1) / 10 * 1e-3) / 1e12
        del a, b
    print(json.dumps(res), flush=True)

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-side", action="store_true",
                    help="decode: leave out the short config-5 prefill and config-4 batched runs of the default line")
    ap.add_argument("--leiden", action="store_true",
                    help="generate: partition every prompt layer with the native Leiden instead of synthetic labels")
    ap.add_argument("--partition-inline", action="store_true",
                    help="generate --leiden: partition each layer inline instead of on the overlapping worker")
    ap.add_argument("--workload", choices=["decode", "prefill", "generate", "batched", "state", "partition", "paper", "floor"],
                    default="decode",
                    help="decode: the 36-layer sparse decode step (default); prefill: config-5 edge export; "
                         "generate: config-3 model decode loop; batched: config-4 ragged batch; "
                         "state: GPU state assembly of one config-2 layer from labels; "
                         "paper: the paper's 131k per-query-head decode setting")
    ap.add_argument("--gen-layers", type=int, default=GEN_LAYERS)
    ap.add_argument("--gen-prompt", type=int, default=GEN_PROMPT)
    ap.add_argument("--gen-steps", type=int, default=GEN_STEPS)
    ap.add_argument("--prefill-seq", type=int, default=PREFILL_SEQ)
    ap.add_argument("--copy-probe", action="store_true",
                    help="after timing, one plain 256 MiB device-to-device copy (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)
    device = torch.device("cuda:0")
    if args.workload == "prefill":
        run_prefill(args, device)
        return
    if args.workload == "generate":
        run_generate(args, device)
        return
    if args.workload == "partition":
        return run_partition(args, device)
    if args.workload == "state":
        return run_state(args, device)
    if args.workload == "batched":
        run_batched(args, device)
        return
    if args.workload == "paper":
        run_paper(args, device)
        return
    if args.workload == "floor":
        run_floor(args, device)
        return
    max_decode = args.warmup + args.steps + max(5, args.steps // 2) + 17  # every full step appends one token
    runtime, stack = build_stack(device, args.layers, max_decode, query_sets=QUERY_SETS)
    torch.cuda.synchronize(device)

    # whole step: 36 layer transitions in one graph.  Each layer's online update
    # (read by nothing else in the step) runs inside the next layer's launch on
    # otherwise idle compute units, and the last layer's inside the first
    # layer's launch of the next step, as CommunityKVRuntime.generate's
    # replayed step does: every replay performs 36 updates (the previous
    # step's last, this step's first 35), each before its layer's next
    # selection.  An eager step before the capture leaves the first pending
    # update; the last one is flushed after the timing.
    # The timed steps rotate over QUERY_SETS captured graphs whose layers read
    # different queries, so a (layer, query) pair recurs only every
    # QUERY_SETS steps: 36 x 4 x ~9.4 MB > 1 GB of gathered rows in between,
    # well beyond the 256 MB Infinity Cache.
    def step_carry(pending, qs):
        for e in stack:
            c = e["calls"][qs]
            c.decode_after(pending)
            pending = c
        return pending

    carried = step_carry(None, 0)
    step_graphs = [capture(lambda qs=qs: step_carry(carried, qs), device) for qs in range(QUERY_SETS)]
    for i in range(args.warmup):
        step_graphs[i % QUERY_SETS].replay()
    torch.cuda.synchronize(device)
    ms, step_ms = time_rotation(step_graphs, args.steps, device)
    stack[-1]["call"].update()
    serial_graph = capture(lambda: [e["call"].decode() for e in stack], device)
    serial_graph.replay()
    serial_ms = time_graph(serial_graph, max(5, args.steps // 2), device)
    att_bytes, step_bytes, tokens_per_head, centroid_bytes = algorithmic_bytes(stack)
    overflow = sum(int(e["layer"].workspace.update.overflow.sum().item()) for e in stack)

    # the step's dominant kernel alone: the cooperative selection + attention +
    # merge launch without a pending update, 36 launches per replay, rotating
    # over the query sets; the layers' states are left as the timed step left them
    fused_graphs = [capture(lambda qs=qs: [e["calls"][qs].decode_after(None) for e in stack], device)
                    for qs in range(QUERY_SETS)]
    for g in fused_graphs:
        g.replay()
    fused_ms = time_rotation(fused_graphs, max(12, args.steps), device)[0] / len(stack)

    # dense bf16 decode over the same 32k caches (baseline)
    dense_ms = dense_decode_ms(stack, SEQ, max(5, args.steps // 5), device)

    # torch-ROCm SDPA decode over the same caches (second dense baseline)
    sdpa_q = [e["query"].view(1, HQ, 1, D) for e in stack]
    sdpa_kv = [(e["key"][:, :SEQ].unsqueeze(0), e["value"][:, :SEQ].unsqueeze(0)) for e in stack]

    def sdpa_step():
        for q, (k, v) in zip(sdpa_q, sdpa_kv):
            torch.nn.functional.scaled_dot_product_attention(q, k, v, enable_gqa=True)

    sdpa_us_layer = None
    try:
        sdpa_graph = capture(sdpa_step, device)
        sdpa_graph.replay()
        sdpa_us_layer = time_graph(sdpa_graph, max(5, args.steps // 5), device) * 1e3 / len(stack)
    except RuntimeError as err:  # reported, not fatal: it is a baseline
        print(f"torch SDPA baseline unavailable: {err}", file=sys.stderr)

    us_layer = ms * 1e3 / len(stack)
    dense_us_layer = dense_ms * 1e3 / len(stack)
    fused_bytes = att_bytes + centroid_bytes
    # The dominant kernel of the timed region is the cooperative launch that
    # carries the previous layer's update: the step graphs hold nothing else,
    # so its average duration is the timed step over its 36 launches (HIP
    # events on the launch stream), and its algorithmic bytes are the step's
    # per layer (selection, attention, output and the update's key row and state).
    achieved = step_bytes / (us_layer * 1e-6) / 1e9
    bare_achieved = fused_bytes / (fused_ms * 1e-3) / 1e9
    result = {
        "metric": "sparse_decode_tokens_per_s_32k_qwen3_8b_attention_stack",
        "value": 1e3 / ms,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (Gaussian-mixture keys, Zipf(1.1) community sizes, random-init state)",
        "config": {"workload": "BASELINE config 2 layer x36: Qwen3-8B attention shape, batch 1, ctx 32768, "
                               "512 communities/KV head, budget 2048 + window 128, QUERY_GROUP, delta-Q update",
                   "layers": len(stack), "query_heads": HQ, "kv_heads": HKV, "head_dim": D, "context": SEQ,
                   "token_budget": BUDGET, "local_window": WINDOW, "num_sink": SINKS},
        "us_per_step_layer": us_layer,
        "us_per_step_layer_median": float(np.median(step_ms)) * 1e3 / len(stack),
        "us_per_step_layer_p10_p90": [float(np.percentile(step_ms, 10)) * 1e3 / len(stack),
                                      float(np.percentile(step_ms, 90)) * 1e3 / len(stack)],
        "query_sets": QUERY_SETS,
        "us_per_step_layer_update_inline": serial_ms * 1e3 / len(stack),
        "dense_us_per_step_layer": dense_us_layer,
        "torch_sdpa_us_per_step_layer": sdpa_us_layer,
        "speedup_vs_dense": dense_us_layer / us_layer,
        "select_attend_kernel_us": fused_ms * 1e3,
        "attended_tokens_per_head": tokens_per_head,
        "step_algorithmic_bytes_per_layer": step_bytes,
        "step_hbm_frac": step_bytes / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "overflow_flags": overflow,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": profiled_traffic("traffic_bytes_per_launch_with_update"),
                     "kernel": "select_attend_kernel<e4m3, bf16, OWN, 18> (cooperative: shared centroid scoring, exact "
                               "selection, slot resolution, KV gather + MFMA attention, in-launch split merge; "
                               "each of the timed step's launches also runs the previous layer's online update)",
                     "bytes_per_launch": step_bytes, "launch_us": us_layer,
                     "timing": "HIP events around the timed step graphs (36 launches each) / 36"},
        "bare_launch": {"us": fused_ms * 1e3, "bytes": fused_bytes, "achieved_gbs": bare_achieved,
                        "frac": bare_achieved / HBM_PEAK_GBS, "traffic": profiled_traffic(),
                        "timing": "graphs of 36 launches without a pending update, rotated over the query sets"},
    }
    if not args.no_side:
        result.update(side_configs(args, device))
    if args.copy_probe:
        src = torch.empty(64 << 20, dtype=torch.int32, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize(device)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(stack[0], args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
