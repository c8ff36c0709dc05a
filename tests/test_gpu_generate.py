"""End-to-end ``CommunityKVRuntime.generate`` on a small random-init Qwen3 model
(reference: runtime.py:510-608, attention/adapter.py:33-81).

With every community selected (``selection="topk"`` over all communities) the
sparse decode attends the whole context, so every step's logits must match a
dense eager forward over the generated sequence up to bf16 rounding; that pins the
plumbing (prefill kernel, edge hand-off, state install, static cache with a
device cursor, deferred online updates, the HIP-graph replay of the
single-token forward, checked on every replayed step) without a reference
run."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

LAYERS = 2
COMMUNITIES = 6


def _model(device):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cfg = Qwen3Config(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=LAYERS,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=8192,
                      rope_theta=1e6, tie_word_embeddings=False)
    torch.manual_seed(0)
    with torch.device(device):
        model = Qwen3ForCausalLM(cfg)
    return model.to(torch.bfloat16).eval()


def _labels(layer_idx, keys, topk_indices, topk_scores):
    graphs, seq_len = keys.shape[0], keys.shape[1]
    g = torch.Generator(device=keys.device).manual_seed(100 + layer_idx)
    lab = torch.randint(0, COMMUNITIES, (graphs, seq_len), generator=g, device=keys.device, dtype=torch.int32)
    lab[:, :10] = 0  # sink positions (ignored)
    lab[:, 10:10 + COMMUNITIES] = torch.arange(COMMUNITIES, device=keys.device, dtype=torch.int32)
    return lab


@pytest.mark.parametrize("assignment,graph,leiden", [("delta_q", True, ""), ("nearest_centroid", True, ""),
                                                     ("delta_q", False, ""), ("delta_q", True, "overlap"),
                                                     ("nearest_centroid", True, "inline")])
def test_generate_full_selection_matches_dense(device, assignment, graph, leiden):
    """``leiden``: no label provider, every prefill layer is partitioned by the
    native Leiden on its top-k edges (build_partitioned_layer), on a worker
    thread and stream overlapping the next layers ("overlap") or inline."""
    from community_kv_amd import CommunityKVAttention, CommunityKVConfig, CommunityKVRuntime, GraphAggregation
    from community_kv_amd.config import PartitionConfig

    print(f"generate e2e assignment={assignment} graph={graph} leiden={leiden}", flush=True)
    model = _model(device)
    prompt = torch.randint(0, 512, (1, 300), generator=torch.Generator().manual_seed(1)).to(device)
    new = 8
    cfg = CommunityKVConfig(token_budget=4096, num_sink=10, aggregation=GraphAggregation.QUERY_GROUP,
                            selection="topk", topk_communities=8192 if leiden else COMMUNITIES,
                            max_selected=4096, assignment=assignment)
    with CommunityKVRuntime(config=cfg, partition=PartitionConfig(overlap=leiden != "inline"), num_layers=LAYERS,
                            max_decode_tokens=new, label_provider=None if leiden else _labels) as runtime:
        CommunityKVAttention(runtime).register()
        model.set_attn_implementation("community_kv")
        with torch.inference_mode():
            out = runtime.generate(model, prompt, max_new_tokens=new, output_logits=True,
                                   return_dict_in_generate=True, graph_decode=graph)
        torch.cuda.synchronize()
        # prefill + one eager decode step, then one graph replay per further token
        assert runtime.last_graph_replays == (new - 2 if graph else 0)
        # every decoded token joined a community of every graph
        for layer in runtime.decode_runtime.layers.values():
            cur = layer.converted.current_position.cpu()
            assert bool((cur == 300 + new - 1).all()), cur
            if leiden:  # Leiden found several communities in every graph
                assert min(layer.converted.initial_community_counts) > 1
    # teacher-forced dense reference over the generated sequence (greedy near-ties
    # cannot make the two runs diverge)
    seq = out.sequences
    assert seq.shape == (1, 300 + new)
    model.set_attn_implementation("eager")
    with torch.inference_mode():
        dense = model(seq[:, :-1]).logits[0, 299:].float()
    for step, a in enumerate(out.logits):
        b = dense[step]
        scale = b.abs().max().item()
        err = (a[0].float() - b).abs().max().item()
        print(f"step {step}: max |logit diff| {err:.4f} (max |logit| {scale:.3f})", flush=True)
        assert err < 0.02 * scale + 0.01, step
        assert int(seq[0, 300 + step]) == int(a[0].argmax())


def test_generate_twice_repeats_itself(device):
    """A second request on the same runtime (state reset, new cache, the step
    graph captured again) reproduces the first one token for token."""
    from community_kv_amd import CommunityKVAttention, CommunityKVConfig, CommunityKVRuntime, GraphAggregation
    from community_kv_amd.config import PartitionConfig

    print("generate twice", flush=True)
    model = _model(device)
    prompt = torch.randint(0, 512, (1, 260), generator=torch.Generator().manual_seed(3)).to(device)
    new = 6
    cfg = CommunityKVConfig(token_budget=128, num_sink=10, aggregation=GraphAggregation.QUERY_GROUP,
                            local_window=32, assignment="delta_q")
    with CommunityKVRuntime(config=cfg, partition=PartitionConfig(), num_layers=LAYERS, max_decode_tokens=new,
                            label_provider=_labels) as runtime:
        CommunityKVAttention(runtime).register()
        model.set_attn_implementation("community_kv")
        with torch.inference_mode():
            a = runtime.generate(model, prompt, max_new_tokens=new)
            b = runtime.generate(model, prompt, max_new_tokens=new)
        torch.cuda.synchronize()
        assert runtime.last_graph_replays == new - 2
    assert torch.equal(a, b)
