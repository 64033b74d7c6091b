"""Fused decode-step indexer: dense scores + exact per-sequence top-K.

The reference times this step as ``_full_score_kernel`` followed by
``torch.topk(scores, K, sorted=False)`` (reference
scripts/benchmark_progressive_dsa.py:117-123), and defines the selection as
``stable_topk`` (metrics.py:9-22).  ``indexer_topk`` runs the whole step as
three HIP launches over the full GPU (scoring with a per-row score histogram,
candidate gather, exact resolve) and returns the stable_topk index set of every
sequence in ascending index order.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .progressive_kernel import HEAD_DIM, HEADS


def _workspace(device: torch.device, stream: int, batch: int, length: int) -> torch.Tensor:
    """Zero-initialised workspace shared by calls on one stream with the same
    batch: each call leaves its histogram zeroed for the next, and calls on a
    stream are ordered.  One buffer per batch, grown geometrically, serves
    every length."""

    need = int(_lib.query("dsa_score_topk_workspace_bytes", batch, length))
    return _lib.workspace("score_topk", device, stream, need, zeroed=True, rows=batch)


def indexer_topk(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    k: int,
    *,
    key_scales: torch.Tensor | None = None,
    return_scores: bool = False,
    return_values: bool = False,
):
    """Top-``k`` key indices of each sequence, int64 ``[B, k]`` ascending.

    queries ``[B, 64, 128]`` bf16/fp16, weights ``[B, 64]``, keys ``[B, L, 128]``
    of the query dtype, or fp8 e4m3fn with ``key_scales`` ``[B, ceil(L/128)]``
    (bf16 queries).  Sequences shorter than ``k`` are padded with -1.
    """

    _lib.load()
    if queries.ndim == 2:
        queries, weights, keys = queries[None], weights[None], keys[None]
        if key_scales is not None:
            key_scales = key_scales[None]
    if queries.ndim != 3 or queries.shape[1:] != (HEADS, HEAD_DIM):
        raise ValueError("queries must be [batch,64,128]")
    batch = queries.shape[0]
    if weights.shape != (batch, HEADS):
        raise ValueError("weights must be [batch,64]")
    if keys.ndim != 3 or keys.shape[0] != batch or keys.shape[2] != HEAD_DIM:
        raise ValueError("keys must be [batch,L,128]")
    if not (queries.is_cuda and weights.is_cuda and keys.is_cuda):
        raise ValueError("HIP kernels require GPU tensors")
    length = keys.shape[1]
    if length == 0 or k <= 0:
        raise ValueError("need at least one key and k > 0")
    if keys.dtype == torch.float8_e4m3fn:
        if queries.dtype != torch.bfloat16:
            raise ValueError("fp8 keys are scored against BF16 queries")
        if key_scales is None or key_scales.shape != (batch, math.ceil(length / 128)):
            raise ValueError("fp8 keys need key_scales [batch, ceil(L/128)]")
        key_scales = key_scales.to(device=keys.device, dtype=torch.float32).contiguous()
    elif queries.dtype not in (torch.float16, torch.bfloat16) or keys.dtype != queries.dtype:
        raise ValueError("queries and keys must share FP16/BF16 dtype")
    queries = queries.contiguous()
    keys = keys.contiguous()
    weights = weights.to(torch.float32).contiguous()
    device = keys.device
    stream = _lib.stream_of(keys)
    scores = torch.empty((batch, length), device=device, dtype=torch.float32)
    indices = torch.empty((batch, k), device=device, dtype=torch.int64)
    values = torch.empty((batch, k), device=device, dtype=torch.float32) if return_values else None
    ws = _workspace(device, stream, batch, length)
    _lib.call(
        "dsa_score_topk", _lib.ptr(queries), _lib.ptr(weights), _lib.ptr(keys), _lib.ptr(key_scales),
        _lib.ptr(scores), batch, length, k, _lib.dtype_code(keys.dtype), _lib.ptr(indices),
        _lib.ptr(values), _lib.ptr(ws), ws.numel(), stream,
    )
    out = [indices]
    if return_scores:
        out.append(scores)
    if return_values:
        out.append(values)
    return out[0] if len(out) == 1 else tuple(out)
