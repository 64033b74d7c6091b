"""Verifier scores on the GPU: head-sparse and dim-sparse paths, routing.

Mirrors ``temporal_dsa.verifier_scoring`` (reference
``src/temporal_dsa/verifier_scoring.py``): ``normalized_hadamard`` (:9-26),
``fake_symmetric_quantize`` (:29-41), ``score_head_sparse`` (:49-92),
``score_dim_sparse`` (:95-139), ``dynamic_head_indices`` (:142-159) and
``layer_energy_dimensions`` (:162-170).  Dot products accumulate in float32
(the reference's einsum rounds each head's dot to the input dtype; the
kernels keep float32, as the reference's own Triton kernels do).
"""

from __future__ import annotations

import numpy as np
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


def normalized_hadamard(tensor: torch.Tensor) -> torch.Tensor:
    """Orthonormal Walsh-Hadamard transform on the last axis (a power of two
    <= 128), each butterfly stage rounded to the tensor's dtype like the
    reference's tensor arithmetic (verifier_scoring.py:9-26)."""

    from .verifier import dim_sketch

    size = tensor.shape[-1]
    if size <= 0 or size & (size - 1):
        raise ValueError("Hadamard dimension must be a positive power of two")
    return dim_sketch(tensor, torch.arange(size), rotation="hadamard")


def fake_symmetric_quantize(tensor: torch.Tensor, bits: int, scale: float | None = None):
    """(fake-quantized tensor, scale) with a fixed symmetric tensor scale
    (verifier_scoring.py:29-41): scale = max|x| / (2^(bits-1) - 1) unless
    given, at least 1e-12."""

    from .verifier import _tensor_scale, fake_quantize

    if bits not in {2, 4, 8}:
        raise ValueError("bits must be one of 2, 4, 8")
    if not tensor.is_cuda:
        raise ValueError("HIP kernels require GPU tensors")
    if tensor.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError("fake quantization takes fp32, fp16 or bf16 tensors")
    scale = _tensor_scale(tensor.contiguous(), bits) if scale is None else max(float(scale), 1e-12)
    return fake_quantize(tensor, bits, scale), scale


def score_dim_sparse(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    dimension_indices,
    *,
    rotation: str = "none",
    bits: int | None = None,
    query_scale: float | None = None,
    key_scale: float | None = None,
    query_chunk_size: int = 1,
    key_chunk_size: int = 8192,
) -> torch.Tensor:
    """All-head partial-dimension verifier scores, fp32 ``[Q, K]``
    (verifier_scoring.py:95-139).  BF16 queries ``[Q, H, D]`` (H <= 64, D a
    power of two <= 128) and keys ``[K, D]``; the dimension count must be a
    multiple of 8.  The chunk sizes are accepted for API compatibility."""

    from .verifier import dim_sketch

    del query_chunk_size, key_chunk_size
    if queries.ndim != 3 or weights.shape != queries.shape[:2] or keys.ndim != 2:
        raise ValueError("expected queries [Q,H,D], weights [Q,H], keys [K,D]")
    if rotation not in ("none", "hadamard"):
        raise ValueError("rotation must be 'none' or 'hadamard'")
    if not (queries.is_cuda and weights.is_cuda and keys.is_cuda):
        raise ValueError("HIP kernels require GPU tensors")
    if queries.dtype != torch.bfloat16:
        raise ValueError("the sketch kernels take BF16 queries")
    num_queries, heads, dim = queries.shape
    if keys.shape[1] != dim:
        raise ValueError("queries and keys disagree on the head dimension")
    if heads > 64:
        raise ValueError("at most 64 heads are supported")
    dims = torch.as_tensor(dimension_indices, device=queries.device).reshape(-1)
    width = dims.numel()
    if width % 8 or width > 128:
        raise ValueError("the dimension count must be a multiple of 8, at most 128")
    keys = keys.to(queries.dtype)
    q_sketch = dim_sketch(queries, dims, rotation=rotation, bits=bits, scale=query_scale)
    k_sketch = dim_sketch(keys, dims, rotation=rotation, bits=bits, scale=key_scale)
    out = torch.empty((num_queries, keys.shape[0]), device=queries.device, dtype=torch.float32)
    if num_queries == 0 or keys.shape[0] == 0:
        return out
    w = weights.to(torch.float32).contiguous()
    _lib.call(
        "dsa_sketch_scores", _lib.ptr(q_sketch.contiguous()), _lib.ptr(w), num_queries, heads,
        _lib.ptr(k_sketch.contiguous()), 0, 0.0, width, keys.shape[0], _lib.ptr(out), _lib.stream_of(queries),
    )
    return out


def layer_energy_dimensions(queries: torch.Tensor, keys: torch.Tensor, width: int) -> np.ndarray:
    """A fixed dimension subset from validation q/k energy
    (verifier_scoring.py:162-170): the ``width`` dims of largest
    mean(q^2) * mean(k^2), ascending.  A one-off calibration on the host."""

    q = queries.detach().float().cpu().numpy()
    k = keys.detach().float().cpu().numpy()
    energy = (q * q).reshape(-1, q.shape[-1]).mean(axis=0, dtype=np.float32) * (k * k).mean(axis=0, dtype=np.float32)
    return np.sort(np.argsort(-energy, kind="stable")[:width]).astype(np.int64)
