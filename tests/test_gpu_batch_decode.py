"""Batched decode (``ckv_batch_decode``: selection, attention, merge and update
of several items in one launch each) must leave every item's output and graph
state bit-identical to running the items one by one with ``ckv_decode_layer``
(the single-item path is itself checked against the oracle)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from community_kv_amd.attention.kernels._abi import BatchDecode
from oracle import ckv_oracle as co
from oracle import synthetic as syn
from tests import _helpers as h

pytestmark = pytest.mark.gpu

ITEMS = [  # ragged: different contexts and community counts
    dict(seq_len=4096, communities=64),
    dict(seq_len=2500, communities=40),
    dict(seq_len=6000, communities=150),
]


def _item(fx, params, device):
    state, csr, cur, q, k, v = h.to_device(fx, device)
    ws = h.workspace_for(fx, params, device)
    sinks = torch.arange(params.num_sink, dtype=torch.int32, device=device)
    call = ws.call(query=q, key=k, value=v, csr=csr, state=state, sink_positions=sinks, current_position=cur,
                   softmax_scale=params.softmax_scale, lam=params.lam)
    return dict(state=state, cur=cur, q=q, ws=ws, call=call)


# more than 1024 scored rows per head: the batch scores them first on every
# compute unit (score_rows_batch_kernel), the selection loads the scores
ITEMS_LARGE = [
    dict(seq_len=16384, communities=1500),
    dict(seq_len=6000, communities=300),
    dict(seq_len=12000, communities=1100),
]


# more than 8192 scored rows per head: the batch takes the large selection
# (scoring on every compute unit, 1,024 threads per (item, head)), as each
# item's single call does
ITEMS_HUGE = [
    dict(seq_len=49152, communities=12000),
    dict(seq_len=40000, communities=8500),
    dict(seq_len=32768, communities=9000),
]


@pytest.mark.parametrize("aggregation,assignment,group,items", [
    (co.QUERY_GROUP, "delta_q", 4, ITEMS), (co.QUERY_GROUP, "nearest_centroid", 4, ITEMS),
    (co.LAYER_WISE, "delta_q", 2, ITEMS), (co.QUERY_GROUP, "delta_q", 4, ITEMS_LARGE),
    (co.QUERY_GROUP, "delta_q", 4, ITEMS_HUGE), (co.QUERY_GROUP, "nearest_centroid", 4, ITEMS_HUGE)])
def test_batch_decode_matches_single_items(device, aggregation, assignment, group, items):
    print(f"batch decode {aggregation} {assignment} communities={[kw['communities'] for kw in items]}", flush=True)
    params = co.StepParams(group_size=group, num_sink=10, token_budget=512, local_window=64, assignment=assignment)
    qh = 4 * group
    fxs = [syn.build_layer(seed=50 + i, query_heads=qh, kv_heads=4, num_sink=10, max_decode_tokens=16,
                           aggregation=aggregation, **kw) for i, kw in enumerate(items)]
    single = [_item(fx, params, device) for fx in fxs]
    batched = [_item(fx, params, device) for fx in fxs]
    batch = BatchDecode([b["call"] for b in batched])
    rng = np.random.default_rng(9)
    for step in range(8):
        for it in single:
            it["call"].decode()
        batch.decode()
        torch.cuda.synchronize(device)
        for i, (a, b) in enumerate(zip(single, batched)):
            case = f"step {step} item {i}"
            assert torch.equal(a["ws"].attention.output, b["ws"].attention.output), case
            assert torch.equal(a["ws"].attention.lse, b["ws"].attention.lse), case
            assert torch.equal(a["ws"].selection.slot_positions, b["ws"].selection.slot_positions), case
            h.assert_states_equal(h.state_to_numpy(a["state"], a["cur"], True),
                                  h.state_to_numpy(b["state"], b["cur"], True))
        for fx, a, b in zip(fxs, single, batched):
            q = syn.fresh_query(fx, rng)
            a["q"].copy_(h.torch_values(q, fx.dtype, device))
            b["q"].copy_(h.torch_values(q, fx.dtype, device))


def test_batch_rejects_mismatched_items(device):
    params = co.StepParams(group_size=4, num_sink=10, token_budget=512)
    other = co.StepParams(group_size=4, num_sink=10, token_budget=1024)
    fx0 = syn.build_layer(seed=1, query_heads=16, kv_heads=4, seq_len=4096, communities=64, num_sink=10,
                          max_decode_tokens=4, aggregation=co.QUERY_GROUP)
    fx1 = syn.build_layer(seed=2, query_heads=16, kv_heads=4, seq_len=4096, communities=64, num_sink=10,
                          max_decode_tokens=4, aggregation=co.QUERY_GROUP)
    a, b = _item(fx0, params, device), _item(fx1, other, device)
    with pytest.raises(RuntimeError, match="share"):
        BatchDecode([a["call"], b["call"]])
    with pytest.raises(RuntimeError, match="must not share"):
        BatchDecode([a["call"], a["call"]])


def test_batch_with_one_huge_item_matches_single_selection(device):
    """A batch mixing an item above 8192 scored communities with small ones:
    the whole batch takes the large selection and the separate attention,
    while a small item's single call takes the cooperative fused launch, whose
    split partials are summed in another order.  Selections (slot tables,
    descriptors) must be identical; outputs agree within bf16 rounding."""
    params = co.StepParams(group_size=4, num_sink=10, token_budget=512, local_window=64)
    items = [dict(seq_len=49152, communities=12000), dict(seq_len=3000, communities=60),
             dict(seq_len=6000, communities=300)]
    print("batch decode mixed huge/small", flush=True)
    fxs = [syn.build_layer(seed=80 + i, query_heads=16, kv_heads=4, num_sink=10, max_decode_tokens=4,
                           aggregation=co.QUERY_GROUP, **kw) for i, kw in enumerate(items)]
    single = [_item(fx, params, device) for fx in fxs]
    batched = [_item(fx, params, device) for fx in fxs]
    batch = BatchDecode([b["call"] for b in batched])
    for it in single:
        it["call"].decode()
    batch.decode()
    torch.cuda.synchronize(device)
    for i, (a, b) in enumerate(zip(single, batched)):
        sa, sb = a["ws"].selection, b["ws"].selection
        assert torch.equal(sa.slot_positions, sb.slot_positions), i
        assert torch.equal(sa.communities, sb.communities), i
        assert torch.equal(sa.descriptor_counts, sb.descriptor_counts), i
        oa, ob = a["ws"].attention.output.float(), b["ws"].attention.output.float()
        assert (oa - ob).abs().max().item() < 2e-2, i
        assert (a["ws"].attention.lse - b["ws"].attention.lse).abs().max().item() < 1e-4, i


@pytest.mark.parametrize("aggregation,assignment,group,items", [
    (co.QUERY_GROUP, "delta_q", 4, ITEMS_LARGE), (co.QUERY_GROUP, "nearest_centroid", 4, ITEMS_LARGE),
    (co.LAYER_WISE, "delta_q", 2, ITEMS_LARGE), (co.QUERY_GROUP, "delta_q", 4, ITEMS),
    (co.QUERY_GROUP, "delta_q", 4, ITEMS_HUGE)])
def test_deferred_batch_updates_match_inline(device, aggregation, assignment, group, items):
    """Two layers' batches stepped alternately: ``ckv_batch_decode_after_update``
    (each batch's update left pending and run inside the other batch's
    selection launch, or in a launch of its own where that selection has no
    room for it; the last one flushed with ``ckv_batch_online_update``) must
    give outputs, selections and graph state bit-identical to ``ckv_batch_decode``
    with every update inline."""
    print(f"deferred batch {aggregation} {assignment} communities={[kw['communities'] for kw in items]}",
          flush=True)
    params = co.StepParams(group_size=group, num_sink=10, token_budget=512, local_window=64, assignment=assignment)
    qh = 4 * group
    layers = [[syn.build_layer(seed=base + i, query_heads=qh, kv_heads=4, num_sink=10, max_decode_tokens=16,
                               aggregation=aggregation, **kw) for i, kw in enumerate(items)] for base in (50, 70)]
    inline = [[_item(fx, params, device) for fx in fxs] for fxs in layers]
    deferred = [[_item(fx, params, device) for fx in fxs] for fxs in layers]
    inline_b = [BatchDecode([it["call"] for it in lay]) for lay in inline]
    deferred_b = [BatchDecode([it["call"] for it in lay]) for lay in deferred]
    rng = np.random.default_rng(11)

    def check(lay, step, with_state):
        for i, (a, b) in enumerate(zip(inline[lay], deferred[lay])):
            case = f"layer {lay} step {step} item {i}"
            assert torch.equal(a["ws"].attention.output, b["ws"].attention.output), case
            assert torch.equal(a["ws"].attention.lse, b["ws"].attention.lse), case
            assert torch.equal(a["ws"].selection.slot_positions, b["ws"].selection.slot_positions), case
            if with_state:
                h.assert_states_equal(h.state_to_numpy(a["state"], a["cur"], True),
                                      h.state_to_numpy(b["state"], b["cur"], True))

    pending = None
    for step in range(6):
        for lay in range(2):
            inline_b[lay].decode()
            deferred_b[lay].decode_after(pending)
            pending = deferred_b[lay]
        torch.cuda.synchronize(device)
        check(0, step, True)  # layer 0's update ran in layer 1's selection launch
        check(1, step, False)  # layer 1's update is still pending
        for lay in range(2):
            for fx, a, b in zip(layers[lay], inline[lay], deferred[lay]):
                q = syn.fresh_query(fx, rng)
                a["q"].copy_(h.torch_values(q, fx.dtype, device))
                b["q"].copy_(h.torch_values(q, fx.dtype, device))
    pending.update()
    torch.cuda.synchronize(device)
    check(1, "flush", True)


def test_deferred_batch_rejects_shared_state(device):
    params = co.StepParams(group_size=4, num_sink=10, token_budget=512)
    fx = syn.build_layer(seed=3, query_heads=16, kv_heads=4, seq_len=4096, communities=64, num_sink=10,
                         max_decode_tokens=4, aggregation=co.QUERY_GROUP)
    a = _item(fx, params, device)
    batch = BatchDecode([a["call"]])
    with pytest.raises(RuntimeError, match="must not share"):
        batch.decode_after(batch)
