"""GPU parity of the sparse decode step against the CPU oracle.

Selection (fp16 scores, descriptors, tile starts, slot positions) and the
online update (every state tensor, bit for bit, with the update fed the
device's own top-8 scores/positions and lse) must match exactly; attention
outputs within 2e-2 (bf16) or 1e-5 (fp32) max-abs of the float64 oracle.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from community_kv_amd.attention.decode import decode_layer
from oracle import ckv_oracle as co
from oracle import numerics as nm
from oracle import synthetic as syn
from tests import _helpers as h

pytestmark = pytest.mark.gpu


def _run_step(fx, params, device, dstate=None, ws=None):
    if dstate is None:
        dstate = h.to_device(fx, device)
    state, csr, cur, q, k, v = dstate
    if ws is None:
        ws = h.workspace_for(fx, params, device)
    sinks = torch.arange(params.num_sink, dtype=torch.int32, device=device)
    out, lse, tks, tkp, assigned = decode_layer(
        query=q, key=k, value=v, csr=csr, state=state, sink_positions=sinks, current_position=cur,
        softmax_scale=params.softmax_scale, lam=params.lam, workspace=ws)
    torch.cuda.synchronize()
    return dstate, ws, out, lse, tks, tkp


def _check_selection(fx_state_before, params, ws, ref):
    sel = ws.selection
    R = fx_state_before.retrieval_heads
    scores = sel.scores.cpu().numpy().view(np.uint16)
    for r in range(R):
        count = int(fx_state_before.community_counts[r])
        assert np.array_equal(scores[r, :count], ref.scores[r, :count]), f"fp16 scores differ (head {r})"
        comms, ends = h.descriptor_lists(sel, r)
        assert comms == ref.selections[r].communities, f"descriptor communities differ (head {r})"
        assert ends == list(np.cumsum(ref.selections[r].takes)), f"cumulative ends differ (head {r})"
        assert int(sel.selected_counts[r]) == ref.selections[r].selected_count
        tiles = co.tile_descriptors(ref.selections[r].takes, sel.budget_tiles, params.num_sink)
        assert sel.tile_descriptors[r].cpu().tolist() == tiles.tolist(), f"tile descriptors differ (head {r})"
    slots = sel.slot_positions.cpu().numpy()
    assert np.array_equal(slots, ref.positions), "slot positions differ"


def _check_attention(fx, params, out, lse, ref, dtype):
    tol = 2e-2 if dtype == "bf16" else 1e-5
    got = out.float().cpu().numpy()
    err = np.max(np.abs(got - ref.output))
    assert err <= tol, f"attention output max-abs error {err} > {tol}"
    lse_err = np.max(np.abs(lse.cpu().numpy() - ref.lse))
    assert lse_err <= (1e-3 if dtype == "bf16" else 1e-5), f"lse error {lse_err}"


CASES = {
    # name: (builder kwargs, step params)
    "query_group_bf16": (dict(query_heads=16, kv_heads=4, seq_len=4096, communities=64, num_sink=10,
                              max_decode_tokens=24, aggregation=co.QUERY_GROUP),
                         dict(group_size=4, num_sink=10, token_budget=512, local_window=64)),
    "per_query_head_bf16": (dict(query_heads=8, kv_heads=2, seq_len=2048, communities=48, num_sink=10,
                                 max_decode_tokens=24, aggregation=co.PER_QUERY_HEAD),
                            dict(group_size=1, num_sink=10, token_budget=256)),
    "layer_wise_bf16": (dict(query_heads=8, kv_heads=4, seq_len=2048, communities=40, num_sink=10,
                             max_decode_tokens=24, aggregation=co.LAYER_WISE),
                        dict(group_size=2, num_sink=10, token_budget=320, local_window=32)),
    "nearest_centroid_bf16": (dict(query_heads=16, kv_heads=4, seq_len=4096, communities=64, num_sink=10,
                                   max_decode_tokens=24, aggregation=co.QUERY_GROUP),
                              dict(group_size=4, num_sink=10, token_budget=512, local_window=128,
                                   assignment="nearest_centroid")),
    # more than 1024 / 2048 scored communities per head (two / eight per thread in the selection kernel)
    "communities_1500_bf16": (dict(query_heads=8, kv_heads=2, seq_len=16384, communities=1500, num_sink=10,
                                   max_decode_tokens=8, aggregation=co.QUERY_GROUP),
                              dict(group_size=4, num_sink=10, token_budget=2048, local_window=128)),
    "communities_2600_nearest": (dict(query_heads=4, kv_heads=1, seq_len=16384, communities=2600, num_sink=10,
                                      max_decode_tokens=8, aggregation=co.QUERY_GROUP),
                                 dict(group_size=4, num_sink=10, token_budget=1024, local_window=64,
                                      assignment="nearest_centroid")),
    # more than 8192 scored communities per head: scoring on every compute unit,
    # then the multi-kernel selection (the reference selector's 65,536-community range)
    "communities_12000_bf16": (dict(query_heads=8, kv_heads=2, seq_len=49152, communities=12000, num_sink=10,
                                    max_decode_tokens=8, aggregation=co.QUERY_GROUP),
                               dict(group_size=4, num_sink=10, token_budget=2048, local_window=128)),
    "communities_40000_nearest": (dict(query_heads=4, kv_heads=1, seq_len=98304, communities=40000, num_sink=10,
                                       max_decode_tokens=8, aggregation=co.QUERY_GROUP),
                                  dict(group_size=4, num_sink=10, token_budget=4096, local_window=256,
                                       assignment="nearest_centroid")),
    # 32 per-query-head graphs of 1,500 communities, budget 2,048: separate
    # selection (scoring on every compute unit) and attention launches
    "per_query_head_1500_separate": (dict(query_heads=32, kv_heads=8, seq_len=16384, communities=1500,
                                          num_sink=10, max_decode_tokens=8, aggregation=co.PER_QUERY_HEAD),
                                     dict(group_size=1, num_sink=10, token_budget=2048, local_window=64)),
    # few live communities but 10,000 decode tokens of headroom: a community
    # capacity (10,064) above the single-workgroup selection's 8,192 rows,
    # while only the 64 live rows are scored
    "headroom_10000_bf16": (dict(query_heads=8, kv_heads=2, seq_len=2048, communities=64, num_sink=10,
                                 max_decode_tokens=10000, aggregation=co.QUERY_GROUP),
                            dict(group_size=4, num_sink=10, token_budget=512, local_window=32)),
    # few large communities: decode deltas pile up in a few chains of several geometric chunks
    "deep_delta_chains_bf16": (dict(query_heads=8, kv_heads=2, seq_len=2048, communities=6, num_sink=10,
                                    max_decode_tokens=40, aggregation=co.QUERY_GROUP),
                               dict(group_size=4, num_sink=10, token_budget=512, local_window=32)),
    # every community selected whole (the context is attended in full) while
    # nearest-centroid decode tokens pile into a few communities' chains
    "topk_all_nearest_bf16": (dict(query_heads=8, kv_heads=2, seq_len=300, communities=6, num_sink=10,
                                   max_decode_tokens=12, aggregation=co.QUERY_GROUP),
                              dict(group_size=4, num_sink=10, token_budget=4096, mode="topk", topk_communities=6,
                                   max_selected=4096, assignment="nearest_centroid")),
    # no sinks and no window; a query group of 4 (fused path) and of 8 (selection and attention launches)
    "no_sinks_no_window_bf16": (dict(query_heads=8, kv_heads=2, seq_len=2048, communities=30, num_sink=0,
                                     max_decode_tokens=16, aggregation=co.QUERY_GROUP),
                                dict(group_size=4, num_sink=0, token_budget=256, local_window=0)),
    "group8_bf16": (dict(query_heads=16, kv_heads=2, seq_len=2048, communities=30, num_sink=10,
                         max_decode_tokens=16, aggregation=co.QUERY_GROUP),
                    dict(group_size=8, num_sink=10, token_budget=320, local_window=64)),
}
STEPS = {"headroom_10000_bf16": 3, "communities_1500_bf16": 4, "per_query_head_1500_separate": 3, "communities_2600_nearest": 4, "communities_12000_bf16": 3,
         "communities_40000_nearest": 3, "deep_delta_chains_bf16": 36,
         "topk_all_nearest_bf16": 12}


@pytest.mark.parametrize("name", list(CASES))
def test_decode_steps_match_oracle(device, name):
    build_kw, step_kw = CASES[name]
    print(f"case {name}", flush=True)
    fx = syn.build_layer(seed=11, **build_kw)
    params = co.StepParams(**step_kw)
    dstate = h.to_device(fx, device)
    ws = h.workspace_for(fx, params, device)
    rng = np.random.default_rng(5)
    steps = STEPS.get(name, 12)
    robust_checks = 0
    for step in range(steps):
        before = fx.state.copy()
        dstate, ws, out, lse, tks, tkp = _run_step(fx, params, device, dstate, ws)
        # selection + attention against the untouched oracle state
        ref = co.decode_step(before.copy(), fx.query, fx.keys, fx.values,
                             co.StepParams(**{**step_kw, "assignment": "none"}))
        _check_selection(before, params, ws, ref)
        _check_attention(fx, params, out, lse, ref, fx.dtype)
        for r in range(before.retrieval_heads):
            if int(before.to_graph[r]) == r:
                h.check_topk(tkp[r].cpu().numpy(), tks[r].cpu().numpy(), _scores0(fx, before, ref, r, params),
                             ref.positions[r], params.num_sink)
        # update un-forced (the oracle's own top-8 and lse) on the first steps: same assignment where robust
        if params.assignment != "none" and step < 3:
            ref_u = co.decode_step(before.copy(), fx.query, fx.keys, fx.values, params)
            robust_checks += _unforced_checks(before, fx, params, ref_u, tkp,
                                              ws.update.assigned_communities.cpu().tolist(), f"step {step}")
        # update, teacher-forced with the device's top-8 and lse: bit-exact state
        co.decode_step(fx.state, fx.query, fx.keys, fx.values, params,
                       gpu_topk=(tks.cpu().numpy(), tkp.cpu().numpy()), gpu_lse=lse.cpu().numpy())
        h.assert_states_equal(h.state_to_numpy(dstate[0], dstate[2], fx.state.fp8), h.oracle_state_dict(fx.state))
        assert ws.update.overflow.cpu().tolist() == [0] * len(fx.state.total_weight)
        # next query
        fx.query = syn.fresh_query(fx, rng)
        dstate[3].copy_(h.torch_values(fx.query, fx.dtype, device))
    if params.assignment != "none":
        assert robust_checks > 0, name


def _robust_assignment(before, fx, params, ref_u):
    """The oracle's un-forced assignment per graph, or None where a 1e-4
    relative perturbation of its top-8 scores / lse can change it."""
    base = ref_u.assigned
    robust = [True] * len(base)
    rng = np.random.default_rng(0)
    for trial in range(4):
        sign = rng.choice([-1.0, 1.0], size=ref_u.topk_scores.shape)
        sc = (ref_u.topk_scores * (1.0 + 1e-4 * sign)).astype(np.float32)
        lse = (ref_u.lse * (1.0 + 1e-4 * (1 if trial % 2 else -1))).astype(np.float32)
        alt = co.decode_step(before.copy(), fx.query, fx.keys, fx.values, params,
                             gpu_topk=(sc, ref_u.topk_positions), gpu_lse=lse)
        for g in range(len(base)):
            robust[g] &= int(alt.assigned[g]) == int(base[g])
    return [int(a) if ok else None for a, ok in zip(base, robust)]


def _unforced_checks(before, fx, params, ref_u, tkp, gpu_assigned, case):
    """The device's assignment of each graph against the oracle run on its own
    float64 top-8 and lse (no teacher forcing), wherever that assignment is
    robust (same top-8 set, unchanged by a 1e-4 perturbation).  Returns the
    number of graphs checked."""
    expect = _robust_assignment(before, fx, params, ref_u)
    checked = 0
    for g, a in enumerate(expect):
        same_set = set(tkp[g].cpu().tolist()) == set(ref_u.topk_positions[g].tolist())
        if a is not None and same_set:
            assert gpu_assigned[g] == a, f"{case} graph {g}: device assigned {gpu_assigned[g]}, oracle {a}"
            checked += 1
    return checked


def _scores0(fx, st, ref, r, params):
    kv = int(st.to_kv[r])
    _, _, s = co.attend(fx.query[r * params.group_size:(r + 1) * params.group_size], fx.keys[kv], fx.values[kv],
                        ref.positions[r], params.softmax_scale)
    return s[0]


def test_config1_fp32_topk_window(device):
    """BASELINE config 1 at its own size: fp32, 1 KV head, G=4, S=4096, 64
    communities, top-8 communities + last-64 window, no sinks/current token."""
    fx = syn.build_layer(seed=1, query_heads=4, kv_heads=1, seq_len=4096, communities=64, num_sink=0,
                         max_decode_tokens=1, aggregation=co.QUERY_GROUP, dtype="f32", fp8=False, zipf=False)
    params = co.StepParams(group_size=4, num_sink=0, token_budget=4096, mode="topk", topk_communities=8,
                           max_selected=2048, local_window=64, include_current=False, assignment="none")
    dstate, ws, out, lse, _, _ = _run_step(fx, params, device)
    ref = co.decode_step(fx.state.copy(), fx.query, fx.keys, fx.values, params)
    _check_selection(fx.state, params, ws, ref)
    _check_attention(fx, params, out, lse, ref, "f32")
    assert len(ref.selections[0].communities) == 8


def test_overflow_flags_and_frozen_cursor(device):
    """Exhausted delta pools raise the reference overflow bits and freeze current_position."""
    fx = syn.build_layer(seed=3, query_heads=8, kv_heads=2, seq_len=1024, communities=16, num_sink=10,
                         max_decode_tokens=2, aggregation=co.QUERY_GROUP)
    params = co.StepParams(group_size=4, num_sink=10, token_budget=256)
    dstate = h.to_device(fx, device)
    ws = h.workspace_for(fx, params, device)
    flags = []
    for step in range(4):
        dstate, ws, out, lse, tks, tkp = _run_step(fx, params, device, dstate, ws)
        co.decode_step(fx.state, fx.query, fx.keys, fx.values, params,
                       gpu_topk=(tks.cpu().numpy(), tkp.cpu().numpy()), gpu_lse=lse.cpu().numpy())
        h.assert_states_equal(h.state_to_numpy(dstate[0], dstate[2], True), h.oracle_state_dict(fx.state))
        flags.append(ws.update.overflow.cpu().tolist())
    assert any(any(f) for f in flags), "expected an overflow once the two-token pools are exhausted"


def test_dense_decode_matches_sdpa(device):
    import ctypes

    from community_kv_amd import _native as nat
    from community_kv_amd.attention.kernels import _abi

    torch.manual_seed(0)
    hq, hkv, s = 32, 8, 3000
    q = torch.randn(hq, 128, device=device, dtype=torch.bfloat16)
    k = torch.randn(hkv, s + 100, 128, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    tiles = -(-s // 64)
    pm = torch.empty(hq, tiles, device=device)
    ps = torch.empty_like(pm)
    pa = torch.empty(hq, tiles, 128, device=device)
    out = torch.empty(hq, 128, device=device, dtype=torch.bfloat16)
    lse = torch.empty(hq, device=device)
    kv = _abi.kv_struct(q, k, v)
    nat.check(nat.lib().ckv_dense_decode(ctypes.byref(kv), s, 1 / 128 ** 0.5, pm.data_ptr(), ps.data_ptr(),
                                         pa.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                         ctypes.c_void_p(nat.stream_handle(device))))
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.float().view(1, hkv, 4, 128), k[:, :s].float().unsqueeze(0), v[:, :s].float().unsqueeze(0),
        scale=1 / 128 ** 0.5).reshape(hq, 128)
    assert (out.float() - ref).abs().max().item() < 2e-2
