"""Block key-norm summaries and the certified temporal radius on the GPU.

Mirrors ``temporal_dsa.certified`` (reference ``src/temporal_dsa/certified.py``)
for the two functions that feed pruning bounds: ``block_key_norms``
(certified.py:51-62) and ``temporal_score_radius`` (certified.py:18-48).  The
reference's float64 score oracle ``relu_index_score`` is a test oracle and
lives in ``oracle/``.  Both compute in float64 and return float64, as the
reference does; the radius is rounded up so that it never falls below the
reference's float64 value.
"""

from __future__ import annotations

import math

import torch

from . import _lib


def block_key_norms(keys: torch.Tensor, block_size: int) -> torch.Tensor:
    """Maximum key L2 norm per block and head for keys ``[tokens, heads, dim]``.

    A shared-key cache ``[tokens, dim]`` is treated as one head.
    """

    if not keys.is_cuda:
        raise ValueError("HIP kernels require GPU tensors")
    if keys.ndim == 2:
        keys = keys.unsqueeze(1)
    if keys.ndim != 3:
        raise ValueError("keys must have shape [tokens,heads,dim]")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    tokens, heads, dim = keys.shape
    keys = keys.contiguous()
    blocks = (tokens + block_size - 1) // block_size
    out = torch.empty((blocks, heads), device=keys.device, dtype=torch.float64)
    if tokens == 0:
        return out
    _lib.call(
        "dsa_block_key_norms", _lib.ptr(keys), tokens, heads, dim, block_size,
        _lib.dtype_code(keys.dtype), _lib.ptr(out), _lib.stream_of(keys),
    )
    return out


def temporal_score_radius(
    q_now: torch.Tensor,
    q_prev: torch.Tensor,
    w_now: torch.Tensor,
    w_prev: torch.Tensor,
    block_key_norm: torch.Tensor,
) -> torch.Tensor:
    """Certified |I_t - I_(t-1)| radius for every key block, float64 ``[blocks]``.

    radius_b = sum_h norm[b,h] * (|w_now-w_prev|_h ||q_prev,h|| + |w_now|_h ||q_now,h-q_prev,h||)
    (reference certified.py:43-47), evaluated in float64 and scaled by
    (1 + 2^-36) so that it is never below the reference's float64 value.
    """

    tensors = (q_now, q_prev, w_now, w_prev, block_key_norm)
    if not all(t.is_cuda for t in tensors):
        raise ValueError("HIP kernels require GPU tensors")
    if q_now.shape != q_prev.shape or q_now.ndim != 2:
        raise ValueError("query tensors must have shape [heads,dim]")
    if w_now.shape != w_prev.shape or w_now.shape != (q_now.shape[0],):
        raise ValueError("weight tensors must have shape [heads]")
    if block_key_norm.ndim != 2 or block_key_norm.shape[1] != q_now.shape[0]:
        raise ValueError("block_key_norm must have shape [blocks,heads]")
    heads, dim = q_now.shape
    if heads > 1024 or dim + heads > 8188:
        raise ValueError("temporal_score_radius supports heads <= 1024 and dim + heads <= 8188")
    f64 = [t.to(torch.float64).contiguous() for t in tensors]
    out = torch.empty(block_key_norm.shape[0], device=q_now.device, dtype=torch.float64)
    if out.numel() == 0:
        return out
    _lib.call(
        "dsa_temporal_score_radius", *(_lib.ptr(t) for t in f64), block_key_norm.shape[0], heads,
        dim, _lib.ptr(out), _lib.stream_of(q_now),
    )
    return out


def certified_margins(
    q_now: torch.Tensor,
    q_prev: torch.Tensor,
    w_now: torch.Tensor,
    w_prev: torch.Tensor,
    keys: torch.Tensor,
    previous_length: int,
    block_size: int,
    *,
    key_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Certified per-block margins ``[B, ceil(previous_length / block_size)]``
    (float64) of a temporal step over shared-key caches.

    The reference's radius (certified.py:43-47) with every head's block norm
    equal to the block's largest key norm, plus an allowance for the fp32
    rounding of both steps' scores; with the previous step's dense block
    maxima, ``temporal_step(..., block_margins=...)`` then keeps every key of
    the dense top-k.  queries ``[B, 64, 128]`` and keys ``[B, C, 128]``
    (bf16/fp16, the first ``previous_length`` keys are summarised; or fp8
    e4m3fn keys with ``key_scales`` ``[B, ceil(C / 128)]`` and bf16 queries, a
    key's norm then being scale * its fp8 norm), weights ``[B, 64]``.
    """

    tensors = (q_now, q_prev, w_now, w_prev, keys)
    if not all(t.is_cuda for t in tensors):
        raise ValueError("HIP kernels require GPU tensors")
    if q_now.ndim != 3 or q_now.shape[1:] != (64, 128) or q_prev.shape != q_now.shape:
        raise ValueError("queries must be [batch,64,128]")
    batch = q_now.shape[0]
    if w_now.shape != (batch, 64) or w_prev.shape != (batch, 64):
        raise ValueError("weights must be [batch,64]")
    if keys.ndim != 3 or keys.shape[0] != batch or keys.shape[2] != 128:
        raise ValueError("keys must be [batch,C,128]")
    if keys.dtype == torch.float8_e4m3fn:
        if q_now.dtype != torch.bfloat16 or q_prev.dtype != torch.bfloat16:
            raise ValueError("fp8 keys are summarised against BF16 queries")
        if key_scales is None or key_scales.shape != (batch, math.ceil(keys.shape[1] / 128)):
            raise ValueError("fp8 keys need key_scales [batch, ceil(capacity/128)]")
        key_scales = key_scales.to(device=keys.device, dtype=torch.float32).contiguous()
    elif keys.dtype not in (torch.bfloat16, torch.float16) or q_now.dtype != keys.dtype or q_prev.dtype != keys.dtype:
        raise ValueError("queries and keys must share FP16/BF16 dtype")
    if not 0 < previous_length <= keys.shape[1]:
        raise ValueError("previous_length outside the key buffer")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    if keys.stride(2) != 1 or keys.stride(1) != 128:
        keys = keys.contiguous()
    key_stride = keys.stride(0) // 128
    blocks = (previous_length + block_size - 1) // block_size
    out = torch.empty((batch, blocks), device=keys.device, dtype=torch.float64)
    qn, qp = q_now.contiguous(), q_prev.contiguous()
    wn, wp = w_now.to(torch.float32).contiguous(), w_prev.to(torch.float32).contiguous()
    _lib.call(
        "dsa_certified_margins", _lib.ptr(qn), _lib.ptr(qp), _lib.ptr(wn), _lib.ptr(wp), _lib.ptr(keys),
        _lib.ptr(key_scales), key_stride,
        batch, previous_length, block_size, _lib.dtype_code(keys.dtype), _lib.ptr(out), _lib.stream_of(keys),
    )
    return out
