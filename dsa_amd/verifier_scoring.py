"""Head-sparse verifier scoring and per-query head routing.

Mirrors the hot-path part of ``temporal_dsa.verifier_scoring`` (reference
``src/temporal_dsa/verifier_scoring.py:49-92`` ``score_head_sparse`` and
``:142-159`` ``dynamic_head_indices``).  The dim-sparse / Hadamard verifier
variants are outside this package.
"""

from __future__ import annotations

import torch

from . import _lib
from .progressive_kernel import HEAD_DIM

_STRATEGIES = {"high_weight": 0, "positive_weight": 1}


def _route_heads(weights: torch.Tensor, width: int, strategy: str, *, int64: bool = False) -> torch.Tensor:
    """Stable top-`width` head ids per row of GPU weights ``[rows, heads]``."""

    if strategy not in _STRATEGIES:
        raise ValueError("strategy must be high_weight or positive_weight")
    weights = weights.to(torch.float32).contiguous()
    rows, heads = weights.shape
    if not 0 < width <= heads:
        raise ValueError("invalid head width")
    out = torch.empty((rows, width), device=weights.device, dtype=torch.int64 if int64 else torch.int32)
    _lib.call(
        "dsa_route_heads", _lib.ptr(weights), rows, heads, width, _STRATEGIES[strategy],
        None if int64 else _lib.ptr(out), _lib.ptr(out) if int64 else None,
        _lib.stream_of(weights),
    )
    return out


def dynamic_head_indices(weights: torch.Tensor, width: int, strategy: str) -> torch.Tensor:
    """Per-query runtime-visible head routing ``[Q, width]`` int64.

    Reference: verifier_scoring.py:142-159 (stable descending argsort of |w|
    or max(w, 0), lower head id first on ties).
    """

    if not 0 < width <= weights.shape[-1]:
        raise ValueError("invalid head width")
    if strategy not in _STRATEGIES:
        raise ValueError("strategy must be high_weight or positive_weight")
    if not weights.is_cuda:
        raise ValueError("HIP kernels require GPU tensors")
    return _route_heads(weights.reshape(-1, weights.shape[-1]), width, strategy, int64=True)


def score_head_sparse(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    head_indices,
    *,
    query_chunk_size: int = 1,
    key_chunk_size: int = 8192,
) -> torch.Tensor:
    """Selected-head full-dimension verifier scores, fp32 ``[Q, K]``.

    Reference: verifier_scoring.py:49-92.  ``head_indices`` is a fixed
    ``[h_v]`` vector or a per-query ``[Q, h_v]`` matrix (h_v <= 64).  The chunk
    sizes are accepted for API compatibility; the kernel needs no chunking.
    """

    del query_chunk_size, key_chunk_size
    if queries.ndim != 3 or weights.shape != queries.shape[:2] or keys.ndim != 2:
        raise ValueError("expected queries [Q,H,D], weights [Q,H], keys [K,D]")
    if not (queries.is_cuda and weights.is_cuda and keys.is_cuda):
        raise ValueError("HIP kernels require GPU tensors")
    num_queries, heads, dim = queries.shape
    if dim != HEAD_DIM or keys.shape[1] != HEAD_DIM:
        raise ValueError("expected 128-dim heads and keys")
    if queries.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("queries must be FP16/BF16")
    ids = torch.as_tensor(head_indices, device=queries.device, dtype=torch.int32)
    if ids.ndim not in {1, 2}:
        raise ValueError("head_indices must be [h_v] or [Q,h_v]")
    if ids.ndim == 2 and ids.shape[0] != num_queries:
        raise ValueError("dynamic head_indices must have one row per query")
    width = ids.shape[-1]
    if not 0 < width <= 64:
        raise ValueError("between 1 and 64 head ids are supported")
    if num_queries == 0 or keys.shape[0] == 0:
        return torch.empty((num_queries, keys.shape[0]), device=queries.device, dtype=torch.float32)
    if bool(((ids < 0) | (ids >= heads)).any()):
        raise ValueError("head index out of range")
    queries = queries.contiguous()
    keys = keys.to(queries.dtype).contiguous()
    weights = weights.to(torch.float32).contiguous()
    ids = ids.contiguous()
    out = torch.empty((num_queries, keys.shape[0]), device=queries.device, dtype=torch.float32)
    _lib.call(
        "dsa_score_queries",
        _lib.ptr(queries), heads * HEAD_DIM, _lib.ptr(weights), heads, _lib.ptr(ids),
        0 if ids.ndim == 1 else width, width, _lib.ptr(keys), 0, num_queries, None, 0,
        _lib.ptr(out), keys.shape[0], num_queries, keys.shape[0], -1,
        _lib.dtype_code(keys.dtype), _lib.stream_of(keys),
    )
    return out
