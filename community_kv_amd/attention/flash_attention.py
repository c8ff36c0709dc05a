"""Prefill attention with top-k edge export (reference: attention/flash_attention.py:23-51).

Runs the library's ``ckv_prefill_attention_topk`` kernel instead of the
patched FlashAttention-3 op; the return tuple keeps the op's layout
``(out, softmax_lse, out_accum, softmax_lse_accum, topk_val, topk_idx)``.
"""

from __future__ import annotations

import ctypes
from typing import Any

import torch

from community_kv_amd import _native as nat

DEFAULT_KAPPA = 8


def prefill_attention_topk(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *, softmax_scale: float,
                           num_sink: int = 10, kappa: int = DEFAULT_KAPPA,
                           raw_scores: bool = False) -> tuple[Any, ...]:
    """Causal GQA attention over q [B=1, S, Hq, 128], k/v [1, S, Hkv, 128] (bf16)
    plus each row's top-``kappa`` columns in [num_sink, row] for rows
    >= num_sink + kappa - 1.  ``topk_val`` holds the reference probability
    exp(s_q * scale - lse) of the quantised score s_q, or s_q itself (the raw
    q.k score to within 1/512) when ``raw_scores``.  Selection is exact per row:
    largest quantised score first, equal scores to the larger column."""
    if query.ndim != 4 or key.ndim != 4 or value.shape != key.shape:
        raise ValueError("prefill expects q [B, S, Hq, 128] and k/v [B, S, Hkv, 128]")
    if query.shape[0] != 1 or key.shape[0] != 1:
        raise ValueError("prefill supports batch size 1")
    if query.shape[-1] != 128 or key.shape[-1] != 128:
        raise ValueError("prefill requires head dimension 128")
    if query.dtype != torch.bfloat16 or key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
        raise TypeError("prefill requires bfloat16 q/k/v")
    if num_sink < 0:
        raise ValueError("exclude_sink_tokens must be non-negative")
    if key.shape[1] != query.shape[1]:
        raise ValueError("prefill requires equal query and key lengths")
    device = nat.require_device(query, key, value)
    query = query.contiguous() if query.stride(-1) != 1 else query
    key = key.contiguous() if key.stride(-1) != 1 else key
    value = value.contiguous() if value.stride() != key.stride() else value
    _, seq_len, heads, _ = query.shape
    kv_heads = key.shape[2]
    skip = max(0, num_sink + kappa - 1)
    rows = max(0, seq_len - skip)
    out = torch.empty_like(query)
    lse = torch.empty((1, heads, seq_len), dtype=torch.float32, device=device)
    topk_val = torch.empty((1, heads, rows, kappa), dtype=torch.float32, device=device)
    topk_idx = torch.empty((1, heads, rows, kappa), dtype=torch.int32, device=device)
    args = nat.PrefillArgs(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), out.data_ptr(), lse.data_ptr(),
        topk_val.data_ptr() if rows else None, topk_idx.data_ptr() if rows else None,
        query.stride(1), query.stride(2), key.stride(1), key.stride(2), out.stride(1), out.stride(2),
        seq_len, heads, kv_heads, num_sink, kappa, rows, skip, 1 if raw_scores else 0, float(softmax_scale), 0.0)
    nat.check(nat.lib().ckv_prefill_attention_topk(ctypes.byref(args),
                                                   ctypes.c_void_p(nat.stream_handle(device))))
    return out, lse, None, None, topk_val, topk_idx


__all__ = ["prefill_attention_topk"]
