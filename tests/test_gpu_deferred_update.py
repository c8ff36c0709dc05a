"""Deferred online update (carried by the next layer's selection launch) must
leave every layer's output and graph state bit-identical to the serial
select -> attend -> update order, for the fused selection + attention launch
and for separate selection and attention launches."""

from __future__ import annotations

import numpy as np
import pytest
import torch

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
    return dict(state=state, cur=cur, q=q, ws=ws, call=call)


SHAPES = {
    # query groups of 4, 64 communities: the cooperative / fused launch
    "small": (dict(query_heads=16, kv_heads=4, seq_len=4096, communities=64, aggregation=co.QUERY_GROUP),
              dict(group_size=4, token_budget=512, local_window=64)),
    # 32 per-query-head graphs of 1,500 communities and a 2,048-token budget:
    # separate launches, the scoring on every compute unit carrying the
    # pending update
    "per_query_head_1500": (dict(query_heads=32, kv_heads=8, seq_len=16384, communities=1500,
                                 aggregation=co.PER_QUERY_HEAD),
                            dict(group_size=1, token_budget=2048, local_window=64)),
}


@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("assignment", ["delta_q", "nearest_centroid"])
def test_deferred_update_matches_serial(device, assignment, fused, shape):
    build_kw, step_kw = SHAPES[shape]
    params = co.StepParams(num_sink=10, assignment=assignment, **step_kw)
    fxs = [syn.build_layer(seed=31 + i, num_sink=10, max_decode_tokens=16, **build_kw) for i in range(3)]
    serial = [_layer(fx, params, device) for fx in fxs]
    deferred = [_layer(fx, params, device) for fx in fxs]
    rng = np.random.default_rng(7)
    for step in range(8):
        print(f"step {step}", flush=True)
        for lay in serial:
            if fused:
                lay["call"].decode()  # fused selection + attention, merge, update
            else:
                lay["call"].score_select()
                lay["call"].attention()
                lay["call"].update()
        pending = None
        for lay in deferred:
            if fused:
                lay["call"].decode_after(pending)
            else:
                lay["call"].score_select_after(pending)
                lay["call"].attention()
            pending = lay["call"]
        pending.update()
        torch.cuda.synchronize(device)
        for i, (a, b) in enumerate(zip(serial, deferred)):
            assert torch.equal(a["ws"].attention.output, b["ws"].attention.output), f"layer {i} output"
            assert torch.equal(a["ws"].attention.lse, b["ws"].attention.lse), f"layer {i} lse"
            h.assert_states_equal(h.state_to_numpy(a["state"], a["cur"], True),
                                  h.state_to_numpy(b["state"], b["cur"], True))
        for fx, a, b in zip(fxs, serial, deferred):
            q = syn.fresh_query(fx, rng)
            a["q"].copy_(h.torch_values(q, fx.dtype, device))
            b["q"].copy_(h.torch_values(q, fx.dtype, device))
