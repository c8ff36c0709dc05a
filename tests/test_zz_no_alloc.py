"""ckv_decode_layer_static (the allocation-free decode entry point) against
ckv_decode_layer with a caller workspace: two identical layers, one decoded
by each entry point, must give bit-identical outputs, top-8, assignments,
overflow flags and graph state, call after call.  A larger layer is decoded
first, then a smaller one (a different scratch layout, so the static exchange
row and counters are cleared in between), then the larger one again."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from community_kv_amd import _native as nat
from oracle import ckv_oracle as co
from oracle import synthetic as syn
from tests import _helpers as h

pytestmark = pytest.mark.gpu


def _layer(fx, params, device):
    state, csr, cur, q, k, v = h.to_device(fx, device)
    ws = h.workspace_for(fx, params, device)
    sinks = torch.arange(params.num_sink, dtype=torch.int32, device=device)
    call = ws.call(query=q, key=k, value=v, csr=csr, state=state, sink_positions=sinks, current_position=cur,
                   softmax_scale=params.softmax_scale, lam=params.lam)
    return dict(state=state, cur=cur, q=q, ws=ws, call=call, sinks=sinks)


def _outputs(fx, device):
    hq, r, graphs = fx.query.shape[0], fx.state.retrieval_heads, len(fx.state.total_weight)
    return dict(output=torch.empty(hq, 128, dtype=torch.bfloat16, device=device),
                lse=torch.empty(hq, dtype=torch.float32, device=device),
                topk_scores=torch.empty(r, 8, dtype=torch.float32, device=device),
                topk_positions=torch.empty(r, 8, dtype=torch.int32, device=device),
                assigned=torch.empty(graphs, dtype=torch.int32, device=device),
                overflow=torch.zeros(graphs, dtype=torch.int32, device=device))


def _static_decode(lay, out, device):
    c = lay["call"]
    lib = nat.lib()
    need = lib.ckv_decode_static_scratch_bytes(ctypes.byref(c.state), ctypes.byref(c.config), c.kv.query_heads)
    assert 0 < need <= lib.ckv_decode_static_scratch_limit()
    nat.check(lib.ckv_decode_layer_static(
        ctypes.byref(c.kv), ctypes.byref(c.state), ctypes.byref(c.csr), ctypes.byref(c.deltas),
        ctypes.byref(c.config), out["output"].data_ptr(), out["lse"].data_ptr(), out["topk_scores"].data_ptr(),
        out["topk_positions"].data_ptr(), out["assigned"].data_ptr(), out["overflow"].data_ptr(),
        ctypes.c_void_p(nat.stream_handle(device))))


CASES = [
    # name, query heads, kv heads, context, communities, budget, window, assignment
    ("large", 32, 8, 16384, 400, 1024, 128, "delta_q"),
    ("small", 8, 2, 2048, 40, 256, 32, "nearest_centroid"),
    ("large_again", 32, 8, 16384, 400, 1024, 128, "delta_q"),
]


def test_static_decode_matches_workspace_decode(device):
    rng = np.random.default_rng(11)
    for ci, (name, hq, hkv, seq, comms, budget, window, assignment) in enumerate(CASES):
        print(f"no-alloc case {name}: {hq}/{hkv} heads, {seq} tokens, {comms} communities, budget {budget}",
              flush=True)
        params = co.StepParams(group_size=hq // hkv, num_sink=10, token_budget=budget, local_window=window,
                               assignment=assignment)
        fx = syn.build_layer(seed=70 + ci, query_heads=hq, kv_heads=hkv, seq_len=seq, communities=comms, num_sink=10,
                             max_decode_tokens=8, aggregation=co.QUERY_GROUP)
        ref = _layer(fx, params, device)
        tst = _layer(fx, params, device)
        out = _outputs(fx, device)
        for step in range(3):
            ref["call"].decode()
            _static_decode(tst, out, device)
            torch.cuda.synchronize(device)
            att, upd = ref["ws"].attention, ref["ws"].update
            assert torch.equal(att.output, out["output"]), (name, step, "output")
            assert torch.equal(att.lse, out["lse"]), (name, step, "lse")
            assert torch.equal(att.topk_scores, out["topk_scores"]), (name, step, "topk scores")
            assert torch.equal(att.topk_positions, out["topk_positions"]), (name, step, "topk positions")
            assert torch.equal(upd.assigned_communities, out["assigned"]), (name, step, "assigned")
            assert torch.equal(upd.overflow, out["overflow"]), (name, step, "overflow")
            h.assert_states_equal(h.state_to_numpy(ref["state"], ref["cur"], True),
                                  h.state_to_numpy(tst["state"], tst["cur"], True))
            q = h.torch_values(syn.fresh_query(fx, rng), fx.dtype, device)
            ref["q"].copy_(q)
            tst["q"].copy_(q)


def test_static_decode_rejects_layers_over_the_limit(device):
    """A layer whose workspace exceeds the static scratch fails with CKV_E_LIMIT
    before launching anything."""
    params = co.StepParams(group_size=16, num_sink=10, token_budget=8192, local_window=0)
    fx = syn.build_layer(seed=3, query_heads=256, kv_heads=16, seq_len=9000, communities=100, num_sink=10,
                         max_decode_tokens=4, aggregation=co.QUERY_GROUP)
    lay = _layer(fx, params, device)
    c = lay["call"]
    lib = nat.lib()
    assert lib.ckv_decode_static_scratch_bytes(ctypes.byref(c.state), ctypes.byref(c.config),
                                               c.kv.query_heads) > lib.ckv_decode_static_scratch_limit()
    out = _outputs(fx, device)
    rc = lib.ckv_decode_layer_static(
        ctypes.byref(c.kv), ctypes.byref(c.state), ctypes.byref(c.csr), ctypes.byref(c.deltas),
        ctypes.byref(c.config), out["output"].data_ptr(), out["lse"].data_ptr(), out["topk_scores"].data_ptr(),
        out["topk_positions"].data_ptr(), out["assigned"].data_ptr(), out["overflow"].data_ptr(),
        ctypes.c_void_p(nat.stream_handle(device)))
    assert rc != 0 and b"static decode scratch" in lib.ckv_last_error()


def test_static_decode_captured_and_replayed_between_other_layouts(device):
    """ckv_decode_layer_static captured in a HIP graph: each replay must equal
    ckv_decode_layer on a twin layer, also when eager static calls of another
    layout (other head count and community capacity) run between replays."""
    params = co.StepParams(group_size=4, num_sink=10, token_budget=1024, local_window=128)
    fx = syn.build_layer(seed=91, query_heads=32, kv_heads=8, seq_len=16384, communities=400, num_sink=10,
                         max_decode_tokens=8, aggregation=co.QUERY_GROUP)
    other_params = co.StepParams(group_size=4, num_sink=10, token_budget=256, local_window=32,
                                 assignment="nearest_centroid")
    other_fx = syn.build_layer(seed=92, query_heads=8, kv_heads=2, seq_len=2048, communities=40, num_sink=10,
                               max_decode_tokens=16, aggregation=co.QUERY_GROUP)
    print("no-alloc graph capture: 32/8 heads 16384 tokens between 8/2 heads 2048 tokens", flush=True)
    ref = _layer(fx, params, device)
    tst = _layer(fx, params, device)
    other = _layer(other_fx, other_params, device)
    out = _outputs(fx, device)
    other_out = _outputs(other_fx, device)
    torch.cuda.synchronize(device)
    stream = torch.cuda.Stream(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        _static_decode(tst, out, device)       # warm-up outside the capture (first-call set-up)
        stream.synchronize()
        ref["call"].decode()
        stream.synchronize()
        # the warm-up advanced both layers by one identical step
        with torch.cuda.graph(graph, stream=stream):
            _static_decode(tst, out, device)
    torch.cuda.synchronize(device)
    rng = np.random.default_rng(5)
    for replay in range(3):
        _static_decode(other, other_out, device)          # another layout in between
        torch.cuda.synchronize(device)
        graph.replay()
        ref["call"].decode()
        torch.cuda.synchronize(device)
        att = ref["ws"].attention
        assert torch.equal(att.output, out["output"]), (replay, "output")
        assert torch.equal(att.lse, out["lse"]), (replay, "lse")
        assert torch.equal(att.topk_positions, out["topk_positions"]), (replay, "topk positions")
        assert torch.equal(ref["ws"].update.assigned_communities, out["assigned"]), (replay, "assigned")
        h.assert_states_equal(h.state_to_numpy(ref["state"], ref["cur"], True),
                              h.state_to_numpy(tst["state"], tst["cur"], True))
        q = h.torch_values(syn.fresh_query(fx, rng), fx.dtype, device)
        ref["q"].copy_(q)
        tst["q"].copy_(q)
        torch.cuda.synchronize(device)
