"""Batched / multi-query indexer scoring (``score_encoded``).

Reference: ``LightningIndexerSidecar.score_encoded`` (sidecar.py:89-107):
``[B,Q,H,D] x [B,K,D] -> [B,Q,K]`` fp32, ``ReLU(q.k) * w`` summed over heads.
The sidecar's projections, RoPE and training live upstream of this path and
are not part of this package.

Differences from the reference, all documented at the call:
  * dots stay fp32 (the reference's bf16 einsum rounds each dot to bf16 before
    the ReLU; both agree within the 1e-2 relative bf16 tolerance);
  * ``causal=True`` masks key j of query t unless ``j <= t + causal_offset``
    (masked scores are -inf); the reference has no mask;
  * fp8 e4m3fn keys with one fp32 scale per 128 keys are accepted through
    ``key_scales`` ``[B, ceil(K/128)]``.
"""

from __future__ import annotations

import torch

from . import _lib
from .progressive_kernel import HEAD_DIM, HEADS


def score_encoded(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    *,
    key_chunk_size: int | None = None,
    causal: bool = False,
    causal_offset: int | None = None,
    key_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Indexer scores of every (query, key) pair, fp32 ``[B, Q, K]``.

    ``key_chunk_size`` is accepted for API compatibility; the kernel streams
    keys without materialising per-head dots, so no chunking is needed.
    ``causal_offset`` defaults to ``K - Q`` (the last query sees every key).
    """

    del key_chunk_size
    if queries.ndim != 4 or weights.shape != queries.shape[:-1]:
        raise ValueError("queries must be [batch,query,heads,dim]")
    if keys.ndim != 3 or keys.shape[0] != queries.shape[0]:
        raise ValueError("keys must be [batch,key,dim]")
    batch, num_queries, heads, dim = queries.shape
    length = keys.shape[1]
    if heads != HEADS or dim != HEAD_DIM or keys.shape[2] != HEAD_DIM:
        raise ValueError("expected 64 heads x 128 dims")
    if not (queries.is_cuda and weights.is_cuda and keys.is_cuda):
        raise ValueError("HIP kernels require GPU tensors")
    if queries.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("queries must be FP16/BF16")
    fp8 = keys.dtype == torch.float8_e4m3fn
    if fp8:
        if queries.dtype != torch.bfloat16:
            raise ValueError("fp8 keys are scored against BF16 queries")
        if key_scales is None or key_scales.shape != (batch, (length + 127) // 128):
            raise ValueError("fp8 keys need key_scales [batch, ceil(keys/128)]")
        key_scales = key_scales.to(device=keys.device, dtype=torch.float32).contiguous()
    elif keys.dtype != queries.dtype:
        raise ValueError("queries and keys must share FP16/BF16 dtype")
    if length == 0 or num_queries == 0 or batch == 0:
        return torch.empty((batch, num_queries, length), device=keys.device, dtype=torch.float32)
    queries = queries.contiguous()
    keys = keys.contiguous()
    weights = weights.to(torch.float32).contiguous()
    out = torch.empty((batch, num_queries, length), device=keys.device, dtype=torch.float32)
    offset = -1
    if causal:
        offset = length - num_queries if causal_offset is None else int(causal_offset)
        if offset < 0:
            raise ValueError("causal_offset must be non-negative")
    _lib.call(
        "dsa_score_queries",
        _lib.ptr(queries), HEADS * HEAD_DIM, _lib.ptr(weights), HEADS, None, 0, HEADS,
        _lib.ptr(keys), length, num_queries, _lib.ptr(key_scales), (length + 127) // 128,
        _lib.ptr(out), length, batch * num_queries, length, offset,
        _lib.dtype_code(keys.dtype), _lib.stream_of(keys),
    )
    return out
