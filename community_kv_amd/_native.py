"""ctypes binding of libckv_amd.so (include/ckv_amd.h).

The structures below mirror the C ABI field for field.  Every device call goes
through :func:`lib`, which raises when the library is missing: there is no CPU
fallback anywhere in the product path.
"""

from __future__ import annotations

import ctypes
import functools
import os
import subprocess

import torch

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PACKAGE_DIR)
LIB_PATH = os.path.join(PACKAGE_DIR, "libckv_amd.so")
SOURCES = [os.path.join(PACKAGE_DIR, "csrc", name)
           for name in ("ckv_decode.hip", "ckv_select.hip", "ckv_attend.hip", "ckv_prefill.hip", "ckv_diag.hip",
                                "ckv_state.hip", "ckv_leiden.hip", "ckv_noalloc.hip", "ckv_select_large.hip")]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# Flags for single sources.  The prefill attention takes maxima of MFMA
# results that are finite or -inf: without NaNs to honour, fmaxf needs no
# NaN-quieting moves in front of v_max3_f32.
FILE_FLAGS = {"ckv_prefill.hip": ["-fno-honor-nans"]}

ABI_VERSION = 3

CKV_BF16, CKV_F32, CKV_E4M3 = 0, 1, 2
CKV_SELECT_BUDGET, CKV_SELECT_TOPK = 0, 1
CKV_ASSIGN_NONE, CKV_ASSIGN_DELTA_Q, CKV_ASSIGN_NEAREST = 0, 1, 2

HEAD_DIM = 128
TILE = 64
KAPPA = 8
SCORE_BLOCK = 64
MAX_GROUP = 16
MAX_COMMUNITIES = 65536
MAX_SELECT_ROWS = 8192
MAX_DESCRIPTORS = 4096
MAX_SINKS = 256
MAX_WINDOW = 1024

EXPORTED_SYMBOLS = (
    "ckv_score_select",
    "ckv_segmented_attention",
    "ckv_attention_partials",
    "ckv_decode_layer",
    "ckv_decode_layer_static",
    "ckv_decode_static_scratch_bytes",
    "ckv_decode_static_scratch_limit",
    "ckv_online_update",
    "ckv_score_select_after_update",
    "ckv_decode_step_after_update",
    "ckv_select_attend_partials",
    "ckv_batch_table_bytes",
    "ckv_batch_prepare",
    "ckv_batch_decode",
    "ckv_batch_decode_after_update",
    "ckv_batch_online_update",
    "ckv_batch_attention_partials",
    "ckv_dense_decode",
    "ckv_prefill_attention_topk",
    "ckv_state_workspace_bytes",
    "ckv_label_counts",
    "ckv_build_layer_state",
    "ckv_leiden_workspace_bytes",
    "ckv_batched_leiden",
    "ckv_leiden_test_raise_overflow",
    "ckv_aggregate_coo_workspace_bytes",
    "ckv_aggregate_coo",
    "ckv_densify_workspace_bytes",
    "ckv_densify_count",
    "ckv_densify_apply",
    "ckv_partition_modularity_workspace_bytes",
    "ckv_partition_modularity",
    "ckv_adjacency_workspace_bytes",
    "ckv_adjacency_capacity",
    "ckv_build_adjacency",
    "ckv_host_numerics",
    "ckv_device_numerics",
    "ckv_latency_probe",
    "ckv_abi_version",
    "ckv_last_error",
)

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class KvCache(ctypes.Structure):
    _fields_ = [("query", _p), ("key", _p), ("value", _p), ("head_stride", _i64),
                ("token_stride", _i64), ("capacity", _i64), ("query_heads", _i32),
                ("kv_heads", _i32), ("dtype", _i32), ("reserved", _i32)]


class PrefillCsr(ctypes.Structure):
    _fields_ = [("member_offsets", _p), ("member_positions", _p), ("member_stride", _i64)]


class DeltaChunks(ctypes.Structure):
    _fields_ = [("positions", _p), ("chunk_start", _p), ("chunk_capacity", _p), ("chunk_size", _p),
                ("chunk_next", _p), ("chunk_previous", _p), ("community_head", _p),
                ("community_tail", _p), ("community_sizes", _p), ("next_free_chunk", _p),
                ("next_free_position", _p), ("position_capacity", _i32), ("chunks_per_graph", _i32)]


class GraphState(ctypes.Structure):
    _fields_ = [("centroids", _p), ("community_sizes", _p), ("community_counts", _p),
                ("community_weight", _p), ("total_weight", _p), ("token_communities", _p),
                ("retrieval_to_graph", _p), ("retrieval_to_kv", _p), ("current_position", _p),
                ("token_capacity", _i64), ("retrieval_heads", _i32), ("graph_count", _i32),
                ("community_capacity", _i32), ("centroid_dtype", _i32)]


class DecodeConfig(ctypes.Structure):
    _fields_ = [("sink_positions", _p), ("group_size", _i32), ("num_sink", _i32),
                ("token_budget", _i32), ("selection_mode", _i32), ("topk_communities", _i32),
                ("max_selected", _i32), ("local_window", _i32), ("include_current", _i32),
                ("assignment", _i32), ("score_coverage", _i32), ("softmax_scale", _f32),
                ("lam", _f32)]


class DecodeWorkspace(ctypes.Structure):
    _fields_ = [("scores", _p), ("communities", _p), ("cumulative_ends", _p),
                ("descriptor_counts", _p), ("tile_descriptors", _p), ("selected_counts", _p),
                ("slot_positions", _p), ("exchange", _p), ("nearest", _p),
                ("block_counters", _p), ("partial_max", _p), ("partial_sum", _p),
                ("partial_acc", _p), ("slot_scores", _p), ("output", _p), ("lse", _p),
                ("topk_scores", _p), ("topk_positions", _p), ("assigned", _p), ("overflow", _p),
                ("descriptor_capacity", _i32), ("slot_capacity", _i32), ("budget_tiles", _i32),
                ("score_blocks", _i32)]


class LayerArgs(ctypes.Structure):
    _fields_ = [("kv", ctypes.POINTER(KvCache)), ("state", ctypes.POINTER(GraphState)),
                ("csr", ctypes.POINTER(PrefillCsr)), ("deltas", ctypes.POINTER(DeltaChunks)),
                ("config", ctypes.POINTER(DecodeConfig)), ("ws", ctypes.POINTER(DecodeWorkspace))]


class PrefillArgs(ctypes.Structure):
    _fields_ = [("query", _p), ("key", _p), ("value", _p), ("output", _p), ("lse", _p),
                ("topk_scores", _p), ("topk_indices", _p), ("q_row_stride", _i64),
                ("q_head_stride", _i64), ("k_row_stride", _i64), ("k_head_stride", _i64),
                ("o_row_stride", _i64), ("o_head_stride", _i64), ("seq_len", _i32),
                ("query_heads", _i32), ("kv_heads", _i32), ("num_sink", _i32), ("kappa", _i32),
                ("topk_rows", _i32), ("topk_skip", _i32), ("score_kind", _i32),
                ("softmax_scale", _f32), ("reserved", _f32)]


class StateBuildArgs(ctypes.Structure):
    _fields_ = [("labels", _p), ("keys", _p), ("head_stride", _i64), ("token_stride", _i64),
                ("retrieval_to_graph", _p), ("retrieval_to_kv", _p), ("edge_src", _p), ("edge_dst", _p),
                ("edge_weight", _p), ("edges", _i64), ("graphs", _i32), ("seq_len", _i32), ("num_sink", _i32),
                ("retrieval_heads", _i32), ("kv_heads", _i32), ("key_dtype", _i32), ("centroid_dtype", _i32),
                ("max_communities", _i32), ("community_capacity", _i32), ("token_capacity", _i32),
                ("member_offsets", _p), ("member_positions", _p), ("centroids", _p), ("community_sizes", _p),
                ("community_weight", _p), ("total_weight", _p), ("token_communities", _p), ("workspace", _p),
                ("topk_indices", _p), ("topk_scores", _p), ("topk_heads", _i32), ("topk_rows", _i32),
                ("topk_kappa", _i32), ("topk_group", _i32), ("topk_row0", _i32), ("lam", _f32)]


def build(verbose: bool = False) -> str:
    """Compiles libckv_amd.so for gfx950 in-tree (always recompiles): one
    hipcc process per source file in parallel, then one link."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    sources = [s for s in SOURCES if os.path.exists(s)]
    include = ["-I", os.path.join(REPO_DIR, "include")]
    compile_flags = [f for f in HIP_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="ckv_build_") as tmp:
        objects = [os.path.join(tmp, os.path.basename(src) + ".o") for src in sources]
        cmds = [[HIPCC, *compile_flags, *FILE_FLAGS.get(os.path.basename(src), []), *include, "-c", "-o", obj, src]
                for src, obj in zip(sources, objects)]

        def run(cmd):
            return subprocess.run(cmd, capture_output=True, text=True)

        workers = max(1, min(len(cmds), os.cpu_count() or 1, 16))
        with ThreadPoolExecutor(max_workers=workers) as pool:
            procs = list(pool.map(run, cmds))
        for cmd, proc in zip(cmds, procs):
            if proc.returncode != 0:
                raise RuntimeError(f"hipcc failed ({proc.returncode}) on {cmd[-1]}:\n{proc.stderr[-4000:]}")
        link = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB_PATH + ".tmp", *objects]
        proc = run(link)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc link failed ({proc.returncode}):\n{proc.stderr[-4000:]}")
    os.replace(LIB_PATH + ".tmp", LIB_PATH)
    if verbose:
        for cmd in cmds + [link]:
            print(" ".join(cmd))
    lib.cache_clear()
    return LIB_PATH


@functools.cache
def lib() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
    handle = ctypes.CDLL(LIB_PATH)
    for name in ("ckv_score_select", "ckv_segmented_attention", "ckv_attention_partials", "ckv_decode_layer",
                 "ckv_online_update"):
        fn = getattr(handle, name)
        fn.argtypes = [ctypes.POINTER(KvCache), ctypes.POINTER(GraphState), ctypes.POINTER(PrefillCsr),
                       ctypes.POINTER(DeltaChunks), ctypes.POINTER(DecodeConfig),
                       ctypes.POINTER(DecodeWorkspace), _p]
        fn.restype = ctypes.c_int
    handle.ckv_decode_layer_static.argtypes = [ctypes.POINTER(KvCache), ctypes.POINTER(GraphState),
                                               ctypes.POINTER(PrefillCsr), ctypes.POINTER(DeltaChunks),
                                               ctypes.POINTER(DecodeConfig), _p, _p, _p, _p, _p, _p, _p]
    handle.ckv_decode_layer_static.restype = ctypes.c_int
    handle.ckv_decode_static_scratch_bytes.argtypes = [ctypes.POINTER(GraphState), ctypes.POINTER(DecodeConfig),
                                                       _i32]
    handle.ckv_decode_static_scratch_bytes.restype = ctypes.c_size_t
    handle.ckv_decode_static_scratch_limit.argtypes = []
    handle.ckv_decode_static_scratch_limit.restype = ctypes.c_size_t
    handle.ckv_score_select_after_update.argtypes = [ctypes.POINTER(LayerArgs), ctypes.POINTER(LayerArgs), _p]
    handle.ckv_score_select_after_update.restype = ctypes.c_int
    handle.ckv_decode_step_after_update.argtypes = [ctypes.POINTER(LayerArgs), ctypes.POINTER(LayerArgs), _p]
    handle.ckv_decode_step_after_update.restype = ctypes.c_int
    handle.ckv_select_attend_partials.argtypes = [ctypes.POINTER(LayerArgs), _p]
    handle.ckv_select_attend_partials.restype = ctypes.c_int
    handle.ckv_batch_table_bytes.argtypes = [_i32]
    handle.ckv_batch_table_bytes.restype = ctypes.c_size_t
    handle.ckv_batch_prepare.argtypes = [ctypes.POINTER(LayerArgs), _i32, _p, _p]
    handle.ckv_batch_prepare.restype = ctypes.c_int
    handle.ckv_batch_decode.argtypes = [ctypes.POINTER(LayerArgs), _i32, _p, _p]
    handle.ckv_batch_decode.restype = ctypes.c_int
    handle.ckv_batch_decode_after_update.argtypes = [ctypes.POINTER(LayerArgs), _i32, _p, ctypes.POINTER(LayerArgs),
                                                     _i32, _p, _p]
    handle.ckv_batch_decode_after_update.restype = ctypes.c_int
    handle.ckv_batch_online_update.argtypes = [ctypes.POINTER(LayerArgs), _i32, _p, _p]
    handle.ckv_batch_online_update.restype = ctypes.c_int
    handle.ckv_batch_attention_partials.argtypes = [ctypes.POINTER(LayerArgs), _i32, _p, _p]
    handle.ckv_batch_attention_partials.restype = ctypes.c_int
    handle.ckv_dense_decode.argtypes = [ctypes.POINTER(KvCache), _i32, _f32, _p, _p, _p, _p, _p, _p]
    handle.ckv_dense_decode.restype = ctypes.c_int
    if hasattr(handle, "ckv_prefill_attention_topk"):
        handle.ckv_prefill_attention_topk.argtypes = [ctypes.POINTER(PrefillArgs), _p]
        handle.ckv_prefill_attention_topk.restype = ctypes.c_int
    handle.ckv_state_workspace_bytes.argtypes = [_i32, _i32, _i32, _i32, _i32]
    handle.ckv_state_workspace_bytes.restype = ctypes.c_size_t
    handle.ckv_label_counts.argtypes = [_p, _i32, _i32, _i32, _p, _p]
    handle.ckv_label_counts.restype = ctypes.c_int
    handle.ckv_build_layer_state.argtypes = [ctypes.POINTER(StateBuildArgs), _p]
    handle.ckv_build_layer_state.restype = ctypes.c_int
    handle.ckv_leiden_workspace_bytes.argtypes = [_i64, _i32, _i32]
    handle.ckv_leiden_workspace_bytes.restype = ctypes.c_size_t
    handle.ckv_batched_leiden.argtypes = [_p, _p, _p, _i64, _i32, _i32, _f32, _f32, _i32, _i32, _i32, _p, _p, _p,
                                          _p]
    handle.ckv_batched_leiden.restype = ctypes.c_int
    handle.ckv_leiden_test_raise_overflow.argtypes = [_i32]
    handle.ckv_leiden_test_raise_overflow.restype = None
    handle.ckv_aggregate_coo_workspace_bytes.argtypes = [_i64]
    handle.ckv_aggregate_coo_workspace_bytes.restype = ctypes.c_size_t
    handle.ckv_aggregate_coo.argtypes = [_p, _p, _p, _i64, _p, _i32, _p, _p, _p, _p, _p, _p]
    handle.ckv_aggregate_coo.restype = ctypes.c_int
    handle.ckv_densify_workspace_bytes.argtypes = [_i32, _i32]
    handle.ckv_densify_workspace_bytes.restype = ctypes.c_size_t
    handle.ckv_densify_count.argtypes = [_p, _i32, _i32, _p, _p, _p]
    handle.ckv_densify_count.restype = ctypes.c_int
    handle.ckv_densify_apply.argtypes = [_p, _i32, _i32, _i32, _p, _p, _p]
    handle.ckv_densify_apply.restype = ctypes.c_int
    handle.ckv_partition_modularity_workspace_bytes.argtypes = [_i32]
    handle.ckv_partition_modularity_workspace_bytes.restype = ctypes.c_size_t
    handle.ckv_partition_modularity.argtypes = [_p, _p, _p, _i64, _p, _i32, _f32, _p, _p, _p]
    handle.ckv_partition_modularity.restype = ctypes.c_int
    handle.ckv_adjacency_workspace_bytes.argtypes = [_i32, _i32, _i32, _f32]
    handle.ckv_adjacency_workspace_bytes.restype = ctypes.c_size_t
    handle.ckv_adjacency_capacity.argtypes = [_i32, _i32, _i32, _f32]
    handle.ckv_adjacency_capacity.restype = ctypes.c_int64
    handle.ckv_build_adjacency.argtypes = [_p, _p, _p, _i32, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _p, _p]
    handle.ckv_build_adjacency.restype = ctypes.c_int
    handle.ckv_host_numerics.argtypes = [ctypes.c_int, _p, _p, _i64]
    handle.ckv_host_numerics.restype = ctypes.c_int
    handle.ckv_device_numerics.argtypes = [ctypes.c_int, _p, _p, _i64, _p]
    handle.ckv_device_numerics.restype = ctypes.c_int
    handle.ckv_latency_probe.argtypes = [_i32, _p, _i64, _i32, _i32, _i32, _i32, _p, _p]
    handle.ckv_latency_probe.restype = ctypes.c_int
    handle.ckv_last_error.restype = ctypes.c_char_p
    handle.ckv_abi_version.restype = ctypes.c_int
    if handle.ckv_abi_version() != ABI_VERSION:
        raise RuntimeError("libckv_amd.so ABI version mismatch; rebuild it")
    return handle


def check(rc: int) -> None:
    if rc != 0:
        message = lib().ckv_last_error().decode(errors="replace")
        raise RuntimeError(f"ckv error {rc}: {message}")


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one HIP device; CPU tensors are rejected."""
    device = tensors[0].device
    if device.type != "cuda":
        raise RuntimeError("CommunityKV kernels run on the GPU only (got a CPU tensor)")
    for t in tensors:
        if t.device != device:
            raise ValueError("all tensors must share one device")
    return device


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return CKV_BF16
    if dtype == torch.float32:
        return CKV_F32
    if dtype == torch.float8_e4m3fn:
        return CKV_E4M3
    raise TypeError(f"unsupported dtype {dtype}")
