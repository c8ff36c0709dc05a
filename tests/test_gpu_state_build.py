"""GPU state assembly from labels (``ckv_label_counts`` + ``ckv_build_layer_state``)
against the oracle's restatement of the reference's compute_centroids /
build_member_csr / init_modularity_state (graph/partition.py:382-535): CSR,
sizes, token table and centroids bit for bit (the kernel adds keys in
ascending position order, as the oracle does); modularity weights within
float-summation tolerance (both the reference and this build add them with
float atomics)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from community_kv_amd.graph.kernels.state_build import build_layer_state, label_counts
from oracle import ckv_oracle as co

pytestmark = pytest.mark.gpu


def _labels(rng, graphs, seq_len, maxc, num_sink, zipf=False):
    if zipf:
        w = 1.0 / np.arange(1, maxc + 1) ** 1.1
        ids = rng.choice(maxc, size=(graphs, seq_len), p=w / w.sum())
    else:
        ids = rng.integers(0, maxc, size=(graphs, seq_len))
    ids[:, :num_sink] = rng.integers(0, 3, size=(graphs, num_sink))  # sink labels are ignored
    return ids.astype(np.int32)


def _edges(rng, graphs, seq_len, num_sink, n):
    g = rng.integers(0, graphs, n)
    a = rng.integers(num_sink, seq_len, n)
    b = rng.integers(num_sink, seq_len, n)
    order = np.lexsort((b, a, g))
    src = (g * seq_len + a)[order].astype(np.int32)
    dst = (g * seq_len + b)[order].astype(np.int32)
    w = rng.random(n).astype(np.float32)
    return src, dst, w


CASES = [
    # graphs, seq_len, num_sink, maxc, to_graph, to_kv, key dtype, fp8, zipf, edges
    (2, 5000, 10, 300, [0, 1], [0, 1], torch.bfloat16, True, False, 20000),
    (1, 3000, 4, 40, [0, 0, 0, 0], [0, 1, 2, 3], torch.float32, False, False, 5000),
    (3, 64, 0, 1, [0, 1, 2], [2, 1, 0], torch.bfloat16, True, False, 0),
    (4, 9000, 10, 2000, [0, 1, 2, 3], [0, 1, 2, 3], torch.bfloat16, True, True, 0),
    # more communities than the kernels' LDS counters (16,384): the rest counted in global memory
    (2, 60000, 10, 30000, [0, 1], [0, 1], torch.bfloat16, True, False, 100000),
    # config 2 shape: 8 graphs x 32k positions, 512 Zipf communities, prefill-sized edge list
    (8, 32768, 10, 512, list(range(8)), list(range(8)), torch.bfloat16, True, True, 400000),
]


@pytest.mark.parametrize("graphs,seq_len,num_sink,maxc,to_graph,to_kv,kdt,fp8,zipf,n_edges", CASES)
def test_state_build_matches_oracle(device, graphs, seq_len, num_sink, maxc, to_graph, to_kv, kdt, fp8, zipf,
                                    n_edges):
    print(f"state build graphs={graphs} S={seq_len} sinks={num_sink} maxc={maxc} heads={len(to_graph)} "
          f"{kdt} fp8={fp8} edges={n_edges}", flush=True)
    rng = np.random.default_rng(seq_len + maxc)
    ids = _labels(rng, graphs, seq_len, maxc, num_sink, zipf)
    if graphs > 1:
        ids[-1, num_sink:] %= max(1, maxc // 2)  # graphs with different community counts
    kv_heads = max(to_kv) + 1
    cache = torch.randn(kv_heads, seq_len + 77, 128, generator=torch.Generator().manual_seed(3)) * 2.0
    cache = cache.to(kdt)
    keys = cache.to(device)[:, :seq_len]  # token stride 128, cache longer than the prompt
    edges = _edges(rng, graphs, seq_len, num_sink, n_edges) if n_edges else None
    tg = torch.tensor(to_graph, dtype=torch.int32, device=device)
    tk = torch.tensor(to_kv, dtype=torch.int32, device=device)
    max_decode = 16
    st = build_layer_state(torch.from_numpy(ids).to(device), keys, retrieval_to_graph=tg, retrieval_to_kv=tk,
                           num_sink=num_sink, max_decode_tokens=max_decode, fp8=fp8,
                           edges=None if edges is None else tuple(torch.from_numpy(e).to(device) for e in edges))
    torch.cuda.synchronize()
    counts = (ids[:, num_sink:].max(axis=1) + 1).astype(np.int32)
    assert st.community_counts.cpu().numpy().tolist() == counts.tolist()
    off, pos = co.build_member_csr(ids, counts, num_sink=num_sink)
    np.testing.assert_array_equal(st.member_offsets.cpu().numpy(), off)
    np.testing.assert_array_equal(st.member_positions.cpu().numpy(), pos)
    keys_np = cache[:, :seq_len].float().numpy()
    cent, sizes = co.compute_centroids(ids, counts, keys_np, to_graph=np.asarray(to_graph, np.int32),
                                       to_kv=np.asarray(to_kv, np.int32), num_sink=num_sink,
                                       max_decode_tokens=max_decode, fp8=fp8)
    np.testing.assert_array_equal(st.community_sizes.cpu().numpy(), sizes)
    got = st.centroids.cpu()
    if fp8:
        np.testing.assert_array_equal(got.view(torch.uint8).numpy(), cent)
    else:
        np.testing.assert_array_equal(got.numpy().view(np.uint32), cent.view(np.uint32))
    tok = st.token_communities.cpu().numpy()
    np.testing.assert_array_equal(tok[:, :seq_len], ids)
    assert (tok[:, seq_len:] == -1).all()
    if edges is not None:
        cw, tw = co.init_modularity_state(ids, *edges, community_capacity=st.community_weight.shape[1],
                                          seq_len=seq_len)
        np.testing.assert_allclose(st.community_weight.cpu().numpy(), cw, rtol=2e-5, atol=1e-4)
        np.testing.assert_allclose(st.total_weight.cpu().numpy(), tw, rtol=2e-5)
    else:
        assert not st.community_weight.any() and not st.total_weight.any()


def test_label_counts_flags_negative_labels(device):
    ids = torch.tensor([[5, 1, 2, -3, 0], [7, 7, 0, 1, 4]], dtype=torch.int32, device=device)
    assert label_counts(ids, num_sink=1).cpu().tolist() == [-1, 8]
    assert label_counts(ids, num_sink=4).cpu().tolist() == [1, 5]
    keys = torch.zeros(2, 5, 128, dtype=torch.bfloat16, device=device)
    tg = torch.arange(2, dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="nonnegative"):
        build_layer_state(ids, keys, retrieval_to_graph=tg, retrieval_to_kv=tg, num_sink=1, max_decode_tokens=4)


@pytest.mark.parametrize("lam,kappa", [(0.5, 8), (1.0, 8), (0.3, 16)])
def test_state_build_topk_edges_match_coalesced_graph(device, lam, kappa):
    """Modularity weights from the prefill top-k edges directly must equal
    those of the reference's graph (build_adjacency + init_modularity_state)."""
    from community_kv_amd.graph.kernels.state_build import TopkEdges

    print(f"state build top-k edges lam={lam} kappa={kappa}", flush=True)
    rng = np.random.default_rng(int(lam * 10) + kappa)
    graphs, group, seq_len, num_sink, maxc = 2, 4, 3000, 10, 120
    ids = _labels(rng, graphs, seq_len, maxc, num_sink)
    row0 = num_sink + kappa - 1
    rows = seq_len - row0
    heads = graphs * group
    idx = rng.integers(num_sink, seq_len, size=(heads, rows, kappa)).astype(np.int32)
    idx[rng.random(idx.shape) < 0.05] = -1                 # dropped columns
    idx[rng.random(idx.shape) < 0.02] = seq_len + 3        # outside the sequence
    sc = rng.random((heads, rows, kappa)).astype(np.float32)
    keys = torch.randn(graphs, seq_len, 128, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    tg = torch.arange(graphs, dtype=torch.int32, device=device)
    st = build_layer_state(torch.from_numpy(ids).to(device), keys.to(device), retrieval_to_graph=tg,
                           retrieval_to_kv=tg, num_sink=num_sink, max_decode_tokens=8,
                           topk_edges=TopkEdges(indices=torch.from_numpy(idx).to(device),
                                                scores=torch.from_numpy(sc).to(device), row0=row0, group=group,
                                                lam=lam))
    torch.cuda.synchronize()
    pos = np.tile(np.arange(row0, row0 + rows), group)[None].repeat(graphs, 0)
    src, dst, w = co.build_adjacency(idx.reshape(graphs, group * rows, kappa), sc.reshape(graphs, group * rows, kappa),
                                     pos, seq_len=seq_len, lam=lam)
    cw, tw = co.init_modularity_state(ids, src, dst, w, community_capacity=st.community_weight.shape[1],
                                      seq_len=seq_len)
    np.testing.assert_allclose(st.community_weight.cpu().numpy(), cw, rtol=1e-4, atol=1e-3)
    # the totals add ~10^5-10^6 edge weights: the device's (per-row closed
    # form, per-workgroup partial sums) sits within 1e-5 of the float64 sum;
    # the oracle's one long float32 chain drifts further (checked loosely)
    tw64 = np.array([2.0 * w[src // seq_len == g].astype(np.float64).sum() for g in range(graphs)])
    np.testing.assert_allclose(st.total_weight.cpu().numpy(), tw64, rtol=1e-5)
    np.testing.assert_allclose(tw, tw64, rtol=1e-3)
