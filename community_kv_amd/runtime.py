"""Request runtime: prefill state conversion, per-layer decode, generate().

Reference: community_kv/runtime.py.  ``CommunityKVRuntime`` keeps the
reference constructor, context-manager protocol and ``generate`` contract
(batch 1, greedy, model configured with ``attn_implementation="community_kv"``).
State is validated once per layer in ``prepare_layer``; ``decode`` is a single
native call per layer with no host synchronisation.
"""

from __future__ import annotations

from dataclasses import dataclass
from types import TracebackType
from typing import Any, Mapping, Sequence

import torch

from community_kv_amd.attention.decode import DecodeLayerWorkspace, decode_layer
from community_kv_amd.config import CommunityKVConfig, GraphAggregation, PartitionConfig
from community_kv_amd.graph.partition import PartitionedLayer
from community_kv_amd.graph.runtime import PartitionRuntime
from community_kv_amd.graph.state import DecodeDeltaChunks, MutableGraphState, PrefillCSR

HEAD_DIM = 128
ATTENTION_TILE = 64


def _effective_token_budget(*, configured_budget: int, prefill_seq_len: int, num_sink: int) -> int:
    """The decode budget a prompt can fill exactly (reference runtime.py:22-34):
    the configured budget, capped at the whole 64-slot tiles that the prompt
    plus the current token cover.  Raises when no selected slot would remain
    after the sinks and the current token."""
    whole_tiles = (prefill_seq_len + 1) // ATTENTION_TILE
    budget = min(configured_budget, whole_tiles * ATTENTION_TILE)
    if budget - num_sink - 1 <= 0:
        raise ValueError(f"a {prefill_seq_len}-token prefill is too short for the fixed 64-token decode kernel "
                         f"with {num_sink} sinks (budget {budget})")
    return budget


@dataclass(slots=True)
class ConvertedPrefillState:
    csr: PrefillCSR
    mutable: MutableGraphState
    current_position: torch.Tensor
    initial_community_counts: tuple[int, ...]
    prefill_seq_len: int
    decode_capacity: int
    group_size: int
    aggregation: GraphAggregation
    query_heads: int
    kv_heads: int


@dataclass(slots=True)
class DecodeLayerState:
    converted: ConvertedPrefillState
    workspace: DecodeLayerWorkspace
    sink_positions: torch.Tensor


def _offsets_for_capacity(member_offsets: torch.Tensor, community_capacity: int) -> torch.Tensor:
    """CSR offsets widened to community_capacity + 1 columns: communities that
    decode creates later start empty, at the last prefill offset."""
    if member_offsets.ndim != 2 or member_offsets.dtype != torch.int32:
        raise TypeError(f"member_offsets must be an int32 [graphs, communities + 1] tensor, got "
                        f"{member_offsets.dtype} of rank {member_offsets.ndim}")
    extra = community_capacity + 1 - member_offsets.shape[1]
    if extra < 0:
        raise ValueError(f"member_offsets has {member_offsets.shape[1] - 1} communities, more than the "
                         f"{community_capacity} centroid rows")
    if extra == 0:
        return member_offsets.contiguous()
    return torch.cat([member_offsets, member_offsets[:, -1:].expand(-1, extra)], dim=1).contiguous()


def convert_prefill_tensors(*, member_offsets: torch.Tensor, member_positions: torch.Tensor,
                            num_communities: torch.Tensor, centroids: torch.Tensor, community_sizes: torch.Tensor,
                            community_weight: torch.Tensor, total_weight: torch.Tensor,
                            token_communities: torch.Tensor, retrieval_to_graph: torch.Tensor | None = None,
                            retrieval_to_kv: torch.Tensor | None = None, prefill_seq_len: int,
                            max_decode_tokens: int, group_size: int = 4,
                            aggregation: GraphAggregation = GraphAggregation.PER_QUERY_HEAD,
                            query_heads: int | None = None, kv_heads: int | None = None) -> ConvertedPrefillState:
    """Checks explicit prefill tensors and builds the decode state with empty
    decode-delta pools (reference runtime.py:85-234).

    The layouts are checked by ``PrefillCSR.validate`` and
    ``MutableGraphState.validate`` (dtypes, ranks and shared extents); this
    function adds what only the conversion knows: the head geometry, the
    decode headroom of the token table and the active community counts."""
    if prefill_seq_len <= 0 or max_decode_tokens <= 0:
        raise ValueError(f"prefill_seq_len ({prefill_seq_len}) and max_decode_tokens ({max_decode_tokens}) "
                         "must be positive")
    if not 1 <= group_size <= 16:
        raise ValueError(f"group_size must be in [1, 16], got {group_size}")
    if centroids.ndim != 3 or centroids.shape[-1] != HEAD_DIM or 0 in centroids.shape:
        raise ValueError(f"centroids must be a non-empty [retrieval heads, communities, {HEAD_DIM}] tensor")
    heads, capacity = centroids.shape[0], centroids.shape[1]
    device = centroids.device
    if (retrieval_to_graph is None) != (retrieval_to_kv is None):
        raise ValueError("pass both aggregation mappings or neither")
    if retrieval_to_graph is None:
        if heads != member_offsets.shape[0]:
            raise ValueError("without aggregation mappings every retrieval head needs a graph of its own")
        retrieval_to_graph = retrieval_to_kv = torch.arange(heads, dtype=torch.int32, device=device)
    csr = PrefillCSR(_offsets_for_capacity(member_offsets, capacity), member_positions.contiguous(),
                     num_communities.clone())
    graphs = csr.graph_count
    for name, t in (("retrieval_to_graph", retrieval_to_graph), ("retrieval_to_kv", retrieval_to_kv)):
        if t.dtype != torch.int32 or t.shape != (heads,):
            raise TypeError(f"{name} must be an int32 vector with one entry per retrieval head ({heads})")
    head_counts = num_communities[retrieval_to_graph.long()] if num_communities.shape == (graphs,) else None
    mutable = MutableGraphState(
        centroids=centroids.contiguous(), community_sizes=community_sizes.contiguous(),
        community_counts=(head_counts if head_counts is not None else num_communities).contiguous().clone(),
        community_weight=community_weight.contiguous(), total_weight=total_weight.contiguous(),
        token_communities=token_communities.contiguous(),
        deltas=DecodeDeltaChunks.allocate(graph_count=graphs, community_capacity=capacity,
                                          max_decode_tokens=max_decode_tokens, device=device),
        retrieval_to_graph=retrieval_to_graph.contiguous(), retrieval_to_kv=retrieval_to_kv.contiguous())
    csr.validate()
    mutable.validate()
    if len({t.device for t in (member_offsets, member_positions, num_communities, centroids)}) != 1:
        raise ValueError("the CSR and the graph state must live on one device")
    if token_communities.shape[1] < prefill_seq_len + max_decode_tokens:
        raise ValueError(f"token_communities holds {token_communities.shape[1]} positions; the prefill and the "
                         f"decode headroom need {prefill_seq_len + max_decode_tokens}")
    # head geometry: query heads = retrieval heads x group; KV heads cover the mapping
    highest_kv = int(retrieval_to_kv.max().item())
    query_heads = heads * group_size if query_heads is None else query_heads
    kv_heads = highest_kv + 1 if kv_heads is None else kv_heads
    if query_heads != heads * group_size:
        raise ValueError(f"{query_heads} query heads do not match {heads} retrieval heads x group {group_size}")
    if not 0 <= highest_kv < kv_heads:
        raise ValueError(f"the retrieval heads map to KV head {highest_kv}, beyond the {kv_heads} KV heads")
    initial = tuple(int(c) for c in mutable.community_counts.cpu().tolist())
    if not all(0 < c <= capacity for c in initial):
        raise ValueError(f"active community counts {initial} must lie in [1, {capacity}]")
    current = torch.full((graphs,), prefill_seq_len, dtype=torch.int32, device=device)
    return ConvertedPrefillState(csr, mutable, current, initial, prefill_seq_len, max_decode_tokens, group_size,
                                 GraphAggregation(aggregation), query_heads, kv_heads)


class DecodeRuntime:
    """Fixed-address collection of prepared layer states."""

    def __init__(self, config: CommunityKVConfig, *, defer_updates: bool = False) -> None:
        """``defer_updates``: run each layer's online update inside the next
        decode call's selection launch (idle compute units), which takes it off
        the critical path; ``flush_updates`` runs the last pending one and every
        reader of the graph state calls it first."""
        self.config = config
        self.layers: dict[int, DecodeLayerState] = {}
        self.defer_updates = defer_updates
        self._pending = None  # (layer state, DecodeCall) whose online update has not run yet

    def reset(self) -> None:
        self.layers.clear()
        self._pending = None

    def prepare_partitioned_layer(self, state: PartitionedLayer) -> DecodeLayerState:
        return self.prepare_layer(
            state.layer_idx, member_offsets=state.member_offsets, member_positions=state.member_positions,
            num_communities=state.community_counts, centroids=state.centroids,
            community_sizes=state.community_sizes, community_weight=state.community_weight,
            total_weight=state.total_weight, token_communities=state.token_communities,
            retrieval_to_graph=state.retrieval_to_graph, retrieval_to_kv=state.retrieval_to_kv,
            prefill_seq_len=state.prefill_seq_len,
            max_decode_tokens=state.token_communities.shape[1] - state.prefill_seq_len,
            group_size=state.query_heads // state.retrieval_to_graph.numel(), aggregation=state.aggregation,
            query_heads=state.query_heads, kv_heads=state.kv_heads)

    def prepare_layer(self, layer_idx: int, *, member_offsets, member_positions, num_communities, centroids,
                      community_sizes, community_weight, total_weight, token_communities, retrieval_to_graph=None,
                      retrieval_to_kv=None, prefill_seq_len: int, max_decode_tokens: int, group_size: int = 4,
                      aggregation: GraphAggregation = GraphAggregation.PER_QUERY_HEAD, query_heads=None,
                      kv_heads=None) -> DecodeLayerState:
        if layer_idx in self.layers:
            raise ValueError(f"layer {layer_idx} is already prepared")
        converted = convert_prefill_tensors(
            member_offsets=member_offsets, member_positions=member_positions, num_communities=num_communities,
            centroids=centroids, community_sizes=community_sizes, community_weight=community_weight,
            total_weight=total_weight, token_communities=token_communities, retrieval_to_graph=retrieval_to_graph,
            retrieval_to_kv=retrieval_to_kv, prefill_seq_len=prefill_seq_len, max_decode_tokens=max_decode_tokens,
            group_size=group_size, aggregation=aggregation, query_heads=query_heads, kv_heads=kv_heads)
        mutable = converted.mutable
        cfg = self.config
        budget = _effective_token_budget(configured_budget=cfg.token_budget, prefill_seq_len=prefill_seq_len,
                                         num_sink=cfg.num_sink)
        workspace = DecodeLayerWorkspace.allocate(
            retrieval_head_count=mutable.retrieval_head_count, graph_count=mutable.graph_count,
            group_size=converted.group_size, community_capacity=mutable.community_capacity, token_budget=budget,
            num_sink=cfg.num_sink, dtype=torch.bfloat16, device=mutable.centroids.device,
            score_community_counts=converted.initial_community_counts, score_headroom=max_decode_tokens,
            local_window=cfg.local_window, include_current=cfg.include_current, selection=cfg.selection,
            topk_communities=cfg.topk_communities, max_selected=cfg.max_selected, assignment=cfg.assignment)
        layer = DecodeLayerState(converted, workspace,
                                 torch.arange(cfg.num_sink, dtype=torch.int32, device=mutable.centroids.device))
        self.layers[layer_idx] = layer
        return layer

    def decode(self, *, layer_idx: int, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
               softmax_scale: float) -> torch.Tensor:
        layer = self.layers.get(layer_idx)
        if layer is None:
            raise RuntimeError(f"decode layer {layer_idx} is not prepared")
        if query.ndim != 4 or query.shape[0] != 1 or query.shape[2] != 1 or query.shape[-1] != HEAD_DIM:
            raise ValueError("decode requires query shape [1, Hq, 1, 128]")
        if query.shape[1] != layer.converted.query_heads:
            raise ValueError(f"decode expected {layer.converted.query_heads} query heads, found {query.shape[1]}")
        if key.ndim != 4 or key.shape[0] != 1 or value.shape != key.shape:
            raise ValueError("decode requires key/value shape [1, Hkv, S, 128]")
        if key.shape[1] != layer.converted.kv_heads:
            raise ValueError(f"decode expected {layer.converted.kv_heads} KV heads, found {key.shape[1]}")
        q = query[0, :, 0, :].contiguous()
        if not self.defer_updates:
            output, *_ = decode_layer(
                query=q, key=key[0], value=value[0], csr=layer.converted.csr, state=layer.converted.mutable,
                sink_positions=layer.sink_positions, current_position=layer.converted.current_position,
                softmax_scale=softmax_scale, lam=self.config.lam, workspace=layer.workspace)
            return output.view(1, 1, query.shape[1], HEAD_DIM)
        if self._pending is not None and self._pending[0] is layer:
            self.flush_updates()  # the same layer again: its update must come first
        call = layer.workspace.call(query=q, key=key[0], value=value[0], csr=layer.converted.csr,
                                    state=layer.converted.mutable, sink_positions=layer.sink_positions,
                                    current_position=layer.converted.current_position,
                                    softmax_scale=softmax_scale, lam=self.config.lam)
        call.decode_after(None if self._pending is None else self._pending[1])
        self._pending = (layer, call)
        return layer.workspace.attention.output.view(1, 1, query.shape[1], HEAD_DIM)

    def flush_updates(self) -> None:
        """Runs the pending deferred online update, if any (on the current stream)."""
        if self._pending is not None:
            self._pending[1].update()
            self._pending = None

    def assert_no_overflow(self) -> None:
        self.flush_updates()
        failures = {idx: layer.workspace.update.overflow.detach().cpu().tolist()
                    for idx, layer in self.layers.items()
                    if torch.count_nonzero(layer.workspace.update.overflow).item()}
        if failures:
            raise RuntimeError(f"decode state overflow: {failures}")


class _DecodeStepGraph:
    """Replaces ``model.forward`` during ``CommunityKVRuntime.generate``: every
    single-token step after the first (which completes the prefill hand-off
    and moves the cache cursor to the device) replays one HIP graph of the
    whole model forward -- projections, norms, RoPE, cache writes, the sparse
    decode of every layer with the previous layer's deferred update, and the
    LM head -- instead of launching each kernel from Python.  The step's
    inputs are copied into the graph's fixed buffers; the returned output
    holds the graph's fixed logits buffer (the caller copies what it keeps, as
    ``generate`` does).  Other calls (prefill, first step) run eagerly."""

    def __init__(self, model: Any, runtime: "CommunityKVRuntime") -> None:
        self.model = model
        self.runtime = runtime
        self.forward = model.forward
        self.graph: torch.cuda.CUDAGraph | None = None
        self.static: dict[str, torch.Tensor] = {}
        self.output: Any = None
        self.replays = 0

    # per-step tensors copied into fixed buffers (when the caller passes them;
    # otherwise the model derives positions from the cache's device cursor)
    STEP_TENSORS = ("input_ids", "position_ids", "cache_position")

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        ids = kwargs.get("input_ids")
        if (args or ids is None or ids.ndim != 2 or ids.shape[-1] != 1 or kwargs.get("inputs_embeds") is not None
                or not self.runtime._ready):
            return self.forward(*args, **kwargs)
        if self.graph is None:
            self._capture(kwargs)
        for name in self.STEP_TENSORS:
            if name in self.static:
                self.static[name].copy_(kwargs[name])
        self.graph.replay()
        self.replays += 1
        return self.output

    def _capture(self, kwargs: dict[str, Any]) -> None:
        device = kwargs["input_ids"].device
        self.static = {name: kwargs[name].clone() for name in self.STEP_TENSORS
                       if isinstance(kwargs.get(name), torch.Tensor)}
        call = {k: v for k, v in kwargs.items() if k not in self.STEP_TENSORS and k != "attention_mask"}
        call.update(self.static)
        # the community_kv attention reads no mask, and a 2-D mask grows every step
        call["attention_mask"] = None
        graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream(device)
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.graph(graph, stream=stream):
            self.output = self.forward(**call)
        torch.cuda.current_stream(device).wait_stream(stream)
        self.graph = graph

    def release(self) -> None:
        self.graph = None
        self.output = None
        self.static = {}


class CommunityKVRuntime:
    """Request runtime spanning prefill, partition hand-off and decode (runtime.py:402-614)."""

    def __init__(self, *, config: CommunityKVConfig, partition: PartitionConfig, num_layers: int,
                 max_decode_tokens: int, label_provider=None) -> None:
        if num_layers <= 0 or max_decode_tokens <= 0:
            raise ValueError("num_layers and max_decode_tokens must be positive")
        self.config = config
        self.num_layers = num_layers
        self.max_decode_tokens = max_decode_tokens
        self.decode_runtime = DecodeRuntime(config, defer_updates=True)
        self.partition_runtime = PartitionRuntime(algorithm=config, scheduling=partition, max_layers=num_layers,
                                                  label_provider=label_provider)
        self.resolutions: dict[int, float] = {}
        self._ready = False
        self._generation_cache: Any | None = None

    def __enter__(self) -> "CommunityKVRuntime":
        return self

    def __exit__(self, exc_type: type[BaseException] | None, exc_value: BaseException | None,
                 traceback: TracebackType | None) -> None:
        self.close()

    def start_request(self, *, resolutions: Mapping[int, float] | Sequence[float] | None = None,
                      max_decode_tokens: int | None = None) -> None:
        self.partition_runtime.reset()
        self.decode_runtime.reset()
        self._ready = False
        if max_decode_tokens is not None:
            if max_decode_tokens <= 0:
                raise ValueError("max_decode_tokens must be positive")
            self.max_decode_tokens = max_decode_tokens
        if resolutions is None:
            self.resolutions = {}
        elif isinstance(resolutions, Mapping):
            self.resolutions = {int(k): float(v) for k, v in resolutions.items()}
        else:
            if len(resolutions) != self.num_layers:
                raise ValueError("resolution vector must contain one value per layer")
            self.resolutions = {i: float(v) for i, v in enumerate(resolutions)}
        if any(v <= 0 for v in self.resolutions.values()):
            raise ValueError("all layer resolutions must be positive")

    def submit_prefill_layer(self, *, layer_idx: int, topk_indices: torch.Tensor, topk_scores: torch.Tensor,
                             keys: torch.Tensor, completion_event: Any) -> None:
        self.partition_runtime.submit(
            layer_idx=layer_idx, topk_indices=topk_indices, topk_scores=topk_scores, keys=keys,
            completion_event=completion_event,
            resolution=self.resolutions.get(layer_idx, self.config.leiden_resolution),
            max_decode_tokens=self.max_decode_tokens)

    def finish_prefill(self) -> None:
        if self._ready:
            return
        self.partition_runtime.wait(self.decode_runtime.prepare_partitioned_layer)
        actual = set(self.decode_runtime.layers)
        expected = set(range(self.num_layers))
        if actual != expected:
            raise RuntimeError("partitioned layer set is incomplete: "
                               f"missing={sorted(expected - actual)}, extra={sorted(actual - expected)}")
        self._ready = True
        if self._generation_cache is not None:
            self._generation_cache.enable_device_updates()

    def ensure_ready(self) -> None:
        if not self._ready:
            self.finish_prefill()

    def generate(self, model: Any, inputs: torch.Tensor | None = None, *,
                 resolutions: Mapping[int, float] | Sequence[float] | None = None, **kwargs: Any) -> Any:
        """Generates one sequence with runtime-managed request state and cache (runtime.py:510-608).

        ``graph_decode`` (default True, not a Hugging Face option) replays the
        model's single-token forward from one HIP graph after the first decode
        step (see ``_DecodeStepGraph``); False launches every step eagerly."""
        if inputs is not None and "input_ids" in kwargs:
            raise ValueError("pass input_ids either positionally or by keyword")
        input_ids = kwargs.get("input_ids", inputs)
        if not isinstance(input_ids, torch.Tensor) or input_ids.ndim != 2:
            raise ValueError("generate requires rank-two input_ids")
        if input_ids.shape[0] != 1:
            raise ValueError("CommunityKV generate currently requires batch size 1")
        if getattr(model.config, "_attn_implementation", None) != "community_kv":
            raise ValueError("model.config._attn_implementation must be 'community_kv'")
        for name, message in (("past_key_values", "CommunityKV generate manages past_key_values"),
                              ("cache_implementation", "CommunityKV generate manages the cache implementation"),
                              ("assistant_model", "CommunityKV generate does not support assisted generation"),
                              ("penalty_alpha", "CommunityKV generate does not support contrastive search")):
            if kwargs.get(name) is not None:
                raise ValueError(message)
        if kwargs.get("do_sample") not in (None, False):
            raise ValueError("CommunityKV generate supports greedy decoding only")
        generation_config = kwargs.get("generation_config", getattr(model, "generation_config", None))

        def option(name: str, default: Any) -> Any:
            value = kwargs[name] if name in kwargs else getattr(generation_config, name, default)
            return default if value is None else value  # unset GenerationConfig fields are None

        if option("num_beams", 1) != 1:
            raise ValueError("CommunityKV generate does not support beam search")
        if option("num_return_sequences", 1) != 1:
            raise ValueError("CommunityKV generate supports one returned sequence per prompt")
        prompt_tokens = int(input_ids.shape[-1])
        max_new_tokens = option("max_new_tokens", None)
        if max_new_tokens is None:
            max_length = option("max_length", None)
            if max_length is None:
                raise ValueError("generate requires max_new_tokens or max_length")
            max_new_tokens = int(max_length) - prompt_tokens
        if not isinstance(max_new_tokens, int) or isinstance(max_new_tokens, bool) or max_new_tokens <= 0:
            raise ValueError("max_new_tokens must be a positive integer")
        if int(model.config.num_hidden_layers) != self.num_layers:
            raise ValueError(f"runtime has {self.num_layers} layers but model has {model.config.num_hidden_layers}")
        from community_kv_amd.attention.cache import StaticCache

        cache = StaticCache(num_hidden_layers=self.num_layers, max_cache_len=prompt_tokens + max_new_tokens)
        if getattr(self, "_generation_cache", None) is not None:
            raise RuntimeError("CommunityKV runtime is already generating")
        self.start_request(resolutions=resolutions, max_decode_tokens=max(1, max_new_tokens - 1))
        generate_kwargs = dict(kwargs)
        generate_kwargs.pop("graph_decode", None)
        generate_kwargs.update(past_key_values=cache, do_sample=False, num_beams=1, num_return_sequences=1)
        if hasattr(generation_config, "disable_compile"):
            generate_kwargs["disable_compile"] = True
        self._generation_cache = cache
        step_graph = _DecodeStepGraph(model, self) if kwargs.get("graph_decode", True) else None
        if step_graph is not None:
            model.forward = step_graph
        try:
            output = model.generate(**generate_kwargs) if inputs is None else model.generate(inputs, **generate_kwargs)
            self.finish_prefill()
            self.assert_no_overflow()
            self.last_graph_replays = 0 if step_graph is None else step_graph.replays
            return output
        finally:
            if step_graph is not None:
                del model.forward  # back to the class's forward
                step_graph.release()
            self._generation_cache = None

    def close(self) -> None:
        self.partition_runtime.shutdown()

    def assert_no_overflow(self) -> None:
        self.decode_runtime.assert_no_overflow()


__all__ = ["CommunityKVRuntime", "ConvertedPrefillState", "DecodeLayerState", "DecodeRuntime",
           "convert_prefill_tensors"]
