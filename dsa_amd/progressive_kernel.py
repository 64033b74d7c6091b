"""Indexer scoring entry points with the reference's progressive_kernel API.

Mirrors ``temporal_dsa.progressive_kernel`` (reference
``src/temporal_dsa/progressive_kernel.py``): same names, signatures, defaults,
return types and ``ValueError`` messages, computed by the gfx950 HIP kernels of
``libdsa_amd.so``.  The ``*_triton`` names are kept as aliases of the ``*_hip``
functions so code written against the reference keeps working.

The reference's pure-torch references ``torch_full_scores`` and
``torch_progressive_scores`` are test oracles, not part of this package; their
restatements live in ``oracle/`` next to the tests.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

HEADS = 64
HEAD_DIM = 128
VERIFIER_HEADS = 8
BLOCK_SIZES = (16, 32, 64, 128)


def split_head_ids(selected: torch.Tensor | np.ndarray) -> tuple[torch.Tensor, torch.Tensor]:
    """Selected 8 head ids and their 56-id complement (ascending).

    Reference: progressive_kernel.py:23-34.  Host-side validation of an
    8-element id vector.
    """

    values = torch.as_tensor(selected, dtype=torch.int32)
    if values.is_cuda:
        values = values.cpu()
    if values.ndim != 1 or values.numel() != VERIFIER_HEADS:
        raise ValueError("selected head IDs must have shape [8]")
    if values.min().item() < 0 or values.max().item() >= HEADS:
        raise ValueError("head ID outside [0, 64)")
    if torch.unique(values).numel() != VERIFIER_HEADS:
        raise ValueError("selected head IDs must be unique")
    mask = torch.ones(HEADS, dtype=torch.bool)
    mask[values.long()] = False
    remaining = torch.arange(HEADS, dtype=torch.int32)[mask]
    return values.contiguous(), remaining.contiguous()


def dynamic_head_ids(weights: torch.Tensor, width: int = VERIFIER_HEADS) -> torch.Tensor:
    """Ids of the `width` heads with the largest |w|, ties to the lower id.

    Reference: progressive_kernel.py:37-42.  GPU weights are routed by the HIP
    head-routing kernel; host weights (the reference passes ``weights.cpu()``)
    are ranked on the host like the reference does.
    """

    if weights.shape != (HEADS,):
        raise ValueError("weights must have shape [64]")
    if not 0 < width <= HEADS:
        raise ValueError("invalid head width")
    if weights.is_cuda:
        from .verifier_scoring import _route_heads

        return _route_heads(weights.reshape(1, HEADS), width, "high_weight")[0]
    return torch.argsort(weights.abs(), descending=True, stable=True)[:width].to(torch.int32)


def progressive_qk_reduction(
    length: int,
    direct_full_blocks: int,
    promoted_cold_blocks: int,
    *,
    block_size: int = 64,
) -> float:
    """Fraction of the dense 64-head QK work that the progressive schedule skips.

    Reference: progressive_kernel.py:93-111.
    """

    block_count = math.ceil(length / block_size)
    if min(direct_full_blocks, promoted_cold_blocks) < 0:
        raise ValueError("block counts must be non-negative")
    if direct_full_blocks + promoted_cold_blocks > block_count:
        raise ValueError("accepted block counts exceed total blocks")
    direct_tokens = min(length, direct_full_blocks * block_size)
    promoted_tokens = min(length - direct_tokens, promoted_cold_blocks * block_size)
    cold_tokens = length - direct_tokens
    work = (
        direct_tokens * HEADS
        + cold_tokens * VERIFIER_HEADS
        + promoted_tokens * (HEADS - VERIFIER_HEADS)
    )
    return 1.0 - work / (length * HEADS)


@dataclass(frozen=True)
class ProgressiveResult:
    """Reference: progressive_kernel.py:114-120."""

    scores: torch.Tensor
    accepted_blocks: torch.Tensor
    block_max: torch.Tensor
    candidate_indices: torch.Tensor | None = None
    candidate_count: int | None = None


def _check_gpu_inputs(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    *,
    allow_fp32: bool = False,
    key_scales: torch.Tensor | None = None,
) -> torch.Tensor | None:
    """Input contract of the reference's _check_cuda_inputs (progressive_kernel.py:349-359),
    plus fp8 e4m3fn keys with one fp32 scale per 128 keys (bf16 queries); returns
    the scales ready for the kernels (None for fp16/bf16 keys)."""

    _lib.load()
    if not queries.is_cuda or not weights.is_cuda or not keys.is_cuda:
        raise ValueError("HIP kernels require GPU tensors")
    if queries.shape != (HEADS, HEAD_DIM) or weights.shape != (HEADS,):
        raise ValueError("expected queries [64,128] and weights [64]")
    if keys.ndim != 2 or keys.shape[1] != HEAD_DIM:
        raise ValueError("expected keys [L,128]")
    if keys.shape[0] == 0:
        raise ValueError("expected at least one key")
    if keys.dtype == torch.float8_e4m3fn:
        if queries.dtype != torch.bfloat16:
            raise ValueError("fp8 keys are scored against BF16 queries")
        blocks = (keys.shape[0] + 127) // 128
        if key_scales is None or key_scales.shape != (blocks,):
            raise ValueError(f"fp8 keys need key_scales [{blocks}] (one per 128 keys)")
        return key_scales.to(device=keys.device, dtype=torch.float32).contiguous()
    if key_scales is not None:
        raise ValueError("key_scales apply to fp8 keys only")
    allowed = {torch.float16, torch.bfloat16} | ({torch.float32} if allow_fp32 else set())
    if queries.dtype not in allowed or keys.dtype != queries.dtype:
        raise ValueError("queries and keys must share FP16/BF16 dtype")
    return None


def _check_block_size(block_size: int) -> None:
    if block_size not in BLOCK_SIZES:
        raise ValueError(f"block_size must be one of {BLOCK_SIZES}")


def _weights_f32(weights: torch.Tensor) -> torch.Tensor:
    return weights.to(torch.float32).contiguous()


def _head_ids_on(device: torch.device, ids: torch.Tensor) -> torch.Tensor:
    return ids.to(device=device, dtype=torch.int32).contiguous()


def _mask_bytes(mask: torch.Tensor, device: torch.device) -> torch.Tensor:
    """One byte per block on `device` (bool and int8 are passed through)."""

    mask = mask.to(device)
    if mask.dtype not in (torch.bool, torch.int8, torch.uint8):
        mask = mask != 0
    return mask.contiguous()


def full_scores_hip(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    *,
    block_size: int = 64,
    key_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Dense 64-head indexer score of every key, fp32 ``[L]``.

    Reference: progressive_kernel.py:362-375.  ``block_size`` only selects the
    reference's launch tiling; it is validated and otherwise ignored.  fp32
    queries and keys are accepted as well (fp32 MFMA path), and fp8 e4m3fn keys
    with ``key_scales`` (one fp32 scale per 128 keys) against bf16 queries.
    """

    scales = _check_gpu_inputs(queries, weights, keys, allow_fp32=True, key_scales=key_scales)
    _check_block_size(block_size)
    queries = queries.contiguous()
    keys = keys.contiguous()
    weights = _weights_f32(weights)
    output = torch.empty(keys.shape[0], device=keys.device, dtype=torch.float32)
    _lib.call(
        "dsa_full_scores",
        _lib.ptr(queries), _lib.ptr(weights), _lib.ptr(keys), _lib.ptr(scales), _lib.ptr(output),
        1, keys.shape[0], _lib.dtype_code(keys.dtype), _lib.stream_of(keys),
    )
    return output


def h8_block_max_hip(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    selected_heads: torch.Tensor,
    cold_blocks: torch.Tensor,
    *,
    block_size: int = 64,
    key_scales: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """H8 partial scores (-inf outside cold blocks) and per-block maxima.

    Reference: progressive_kernel.py:378-404 (fp8 keys take ``key_scales`` as
    :func:`full_scores_hip`).
    """

    scales = _check_gpu_inputs(queries, weights, keys, key_scales=key_scales)
    _check_block_size(block_size)
    block_count = math.ceil(keys.shape[0] / block_size)
    if cold_blocks.numel() != block_count:
        raise ValueError("cold block mask length mismatch")
    if selected_heads.is_cuda:
        if selected_heads.numel() != VERIFIER_HEADS:
            raise ValueError("selected head IDs must have shape [8]")
        selected = _head_ids_on(keys.device, selected_heads)
    else:
        selected, _ = split_head_ids(selected_heads)
        selected = _head_ids_on(keys.device, selected)
    queries = queries.contiguous()
    keys = keys.contiguous()
    weights = _weights_f32(weights)
    cold = _mask_bytes(cold_blocks, keys.device)
    partial = torch.empty(keys.shape[0], device=keys.device, dtype=torch.float32)
    maxima = torch.empty(block_count, device=keys.device, dtype=torch.float32)
    _lib.call(
        "dsa_h8_block_max",
        _lib.ptr(queries), _lib.ptr(weights), _lib.ptr(keys), _lib.ptr(scales), _lib.ptr(selected), _lib.ptr(cold),
        _lib.ptr(partial), _lib.ptr(maxima), keys.shape[0], block_size,
        _lib.dtype_code(keys.dtype), _lib.stream_of(keys),
    )
    return partial, maxima


def masked_full_scores_hip(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    keep_blocks: torch.Tensor,
    *,
    block_size: int = 64,
    key_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Full scores on kept blocks, -inf elsewhere (rejected blocks read no keys).

    Reference: progressive_kernel.py:407-424 (fp8 keys take ``key_scales``).
    """

    scales = _check_gpu_inputs(queries, weights, keys, key_scales=key_scales)
    _check_block_size(block_size)
    block_count = math.ceil(keys.shape[0] / block_size)
    if keep_blocks.numel() != block_count:
        raise ValueError("keep block mask length mismatch")
    queries = queries.contiguous()
    keys = keys.contiguous()
    weights = _weights_f32(weights)
    keep = _mask_bytes(keep_blocks, keys.device)
    output = torch.empty(keys.shape[0], device=keys.device, dtype=torch.float32)
    _lib.call(
        "dsa_masked_full_scores",
        _lib.ptr(queries), _lib.ptr(weights), _lib.ptr(keys), _lib.ptr(scales), _lib.ptr(keep), _lib.ptr(output),
        keys.shape[0], block_size, _lib.dtype_code(keys.dtype), _lib.stream_of(keys),
    )
    return output


def progressive_scores_hip(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    selected_heads: torch.Tensor,
    direct_full_blocks: torch.Tensor,
    threshold: float | torch.Tensor,
    *,
    block_size: int = 64,
    compact: bool = False,
    remaining_heads: torch.Tensor | None = None,
    key_scales: torch.Tensor | None = None,
) -> ProgressiveResult:
    """Fused H8 -> promote -> +56 heads scoring.

    Reference: progressive_kernel.py:427-475.  In compact mode the candidate
    count is the exact number of accepted keys (an atomic add of each accepted
    block's valid-key count), so a ragged last block never exposes unwritten
    slots; blocks appear in completion order, keys inside a block in address
    order.  fp8 keys take ``key_scales``; the promotion threshold is compared
    with scaled H8 maxima.
    """

    scales = _check_gpu_inputs(queries, weights, keys, key_scales=key_scales)
    _check_block_size(block_size)
    if remaining_heads is None:
        selected, remaining = split_head_ids(selected_heads)
    else:
        if (
            selected_heads.numel() != VERIFIER_HEADS
            or remaining_heads.numel() != HEADS - VERIFIER_HEADS
        ):
            raise ValueError("expected 8 selected and 56 remaining head IDs")
        selected, remaining = selected_heads, remaining_heads
    selected = _head_ids_on(keys.device, selected)
    remaining = _head_ids_on(keys.device, remaining)
    length = keys.shape[0]
    block_count = math.ceil(length / block_size)
    if direct_full_blocks.numel() != block_count:
        raise ValueError("direct full block mask length mismatch")
    queries = queries.contiguous()
    keys = keys.contiguous()
    weights = _weights_f32(weights)
    direct = _mask_bytes(direct_full_blocks, keys.device)
    threshold_tensor = torch.as_tensor(threshold, device=keys.device, dtype=torch.float32).reshape(1)
    accepted = torch.empty(block_count, device=keys.device, dtype=torch.int8)
    block_max = torch.empty(block_count, device=keys.device, dtype=torch.float32)
    counter = torch.zeros(1, device=keys.device, dtype=torch.int32)
    scores = torch.empty(length, device=keys.device, dtype=torch.float32)
    indices = torch.empty(length, device=keys.device, dtype=torch.int32) if compact else None
    _lib.call(
        "dsa_progressive_scores",
        _lib.ptr(queries), _lib.ptr(weights), _lib.ptr(keys), _lib.ptr(scales), _lib.ptr(selected),
        _lib.ptr(remaining), _lib.ptr(direct), _lib.ptr(threshold_tensor), _lib.ptr(scores),
        _lib.ptr(indices), _lib.ptr(accepted), _lib.ptr(block_max), _lib.ptr(counter),
        length, block_size, int(compact), _lib.dtype_code(keys.dtype), _lib.stream_of(keys),
    )
    candidate_count = None
    if compact:
        candidate_count = int(counter.item())
        scores = scores[:candidate_count]
        assert indices is not None
        indices = indices[:candidate_count]
    return ProgressiveResult(scores, accepted, block_max, indices, candidate_count)


def progressive_scores_batched(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    selected_heads: torch.Tensor,
    direct_full_blocks: torch.Tensor,
    threshold: float | torch.Tensor,
    *,
    block_size: int = 64,
    compact: bool = False,
    key_scales: torch.Tensor | None = None,
) -> ProgressiveResult:
    """:func:`progressive_scores_hip` for ``B`` sequences of one length in
    one launch (``dsa_progressive_scores_batched``).

    queries ``[B, 64, 128]``, weights ``[B, 64]``, keys ``[B, L, 128]`` (fp8
    with ``key_scales`` ``[B, ceil(L/128)]``), selected_heads ``[B, 8]`` (the
    remaining 56 heads of each row are its complement), direct_full_blocks
    ``[B, blocks]``, threshold a float or ``[B]`` tensor.  The result holds
    ``[B, ...]`` tensors; in compact mode ``candidate_indices`` and ``scores``
    are ``[B, L]`` with row b's first ``candidate_count[b]`` entries valid and
    ``candidate_count`` is a device tensor ``[B]`` (no host synchronisation).
    Row b equals :func:`progressive_scores_hip` on sequence b.
    """

    if queries.ndim != 3 or weights.ndim != 2 or keys.ndim != 3:
        raise ValueError("expected queries [B,64,128], weights [B,64] and keys [B,L,128]")
    batch = queries.shape[0]
    if weights.shape[0] != batch or keys.shape[0] != batch:
        raise ValueError("queries, weights and keys must share the batch size")
    if key_scales is not None and (key_scales.ndim != 2 or key_scales.shape[0] != batch):
        raise ValueError("key_scales must be [B, ceil(L/128)]")
    scales = _check_gpu_inputs(queries[0], weights[0], keys[0],
                               key_scales=None if key_scales is None else key_scales[0])
    if scales is not None:
        scales = key_scales.to(device=keys.device, dtype=torch.float32).contiguous()
    _check_block_size(block_size)
    if selected_heads.shape != (batch, VERIFIER_HEADS):
        raise ValueError(f"selected_heads must be [{batch},{VERIFIER_HEADS}]")
    pairs = [split_head_ids(selected_heads[b].cpu()) for b in range(batch)]
    selected = torch.stack([p[0] for p in pairs]).to(device=keys.device, dtype=torch.int32).contiguous()
    remaining = torch.stack([p[1] for p in pairs]).to(device=keys.device, dtype=torch.int32).contiguous()
    length = keys.shape[1]
    block_count = math.ceil(length / block_size)
    if direct_full_blocks.shape != (batch, block_count):
        raise ValueError(f"direct_full_blocks must be [{batch},{block_count}]")
    queries = queries.contiguous()
    keys = keys.contiguous()
    weights = weights.to(torch.float32).contiguous()
    direct = direct_full_blocks.to(device=keys.device, dtype=torch.uint8).contiguous()
    thresholds = torch.as_tensor(threshold, device=keys.device, dtype=torch.float32).reshape(-1)
    if thresholds.numel() == 1:
        thresholds = thresholds.expand(batch)
    if thresholds.numel() != batch:
        raise ValueError("threshold must be a float or one value per sequence")
    thresholds = thresholds.contiguous()
    accepted = torch.empty((batch, block_count), device=keys.device, dtype=torch.int8)
    block_max = torch.empty((batch, block_count), device=keys.device, dtype=torch.float32)
    counters = torch.zeros(batch, device=keys.device, dtype=torch.int32)
    scores = torch.empty((batch, length), device=keys.device, dtype=torch.float32)
    indices = torch.empty((batch, length), device=keys.device, dtype=torch.int32) if compact else None
    _lib.call(
        "dsa_progressive_scores_batched",
        _lib.ptr(queries), _lib.ptr(weights), _lib.ptr(keys), _lib.ptr(scales), _lib.ptr(selected),
        _lib.ptr(remaining), _lib.ptr(direct), _lib.ptr(thresholds), _lib.ptr(scores), _lib.ptr(indices),
        _lib.ptr(accepted), _lib.ptr(block_max), _lib.ptr(counters), batch, length, block_size, int(compact),
        _lib.dtype_code(keys.dtype), _lib.stream_of(keys),
    )
    return ProgressiveResult(scores, accepted, block_max, indices, counters if compact else None)


def two_pass_scores_hip(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    selected_heads: torch.Tensor,
    direct_full_blocks: torch.Tensor,
    threshold: float | torch.Tensor,
    *,
    block_size: int = 64,
    key_scales: torch.Tensor | None = None,
) -> ProgressiveResult:
    """H8 pass, promotion mask, then masked full rerank (three launches).

    Reference: progressive_kernel.py:478-497 (fp8 keys take ``key_scales``).
    """

    _check_gpu_inputs(queries, weights, keys, key_scales=key_scales)
    _check_block_size(block_size)
    direct = _mask_bytes(direct_full_blocks, keys.device)
    cold = (direct == 0) if direct.dtype != torch.bool else ~direct
    _, maxima = h8_block_max_hip(queries, weights, keys, selected_heads, cold, block_size=block_size,
                                 key_scales=key_scales)
    threshold_tensor = torch.as_tensor(threshold, device=keys.device, dtype=torch.float32).reshape(1)
    accepted = torch.empty(maxima.numel(), device=keys.device, dtype=torch.int8)
    _lib.call(
        "dsa_promote_blocks",
        _lib.ptr(direct), _lib.ptr(maxima), _lib.ptr(threshold_tensor), _lib.ptr(accepted),
        maxima.numel(), _lib.stream_of(keys),
    )
    scores = masked_full_scores_hip(queries, weights, keys, accepted, block_size=block_size, key_scales=key_scales)
    return ProgressiveResult(scores, accepted, maxima)


# Reference names (the reference's tests and benchmarks import these).
full_scores_triton = full_scores_hip
h8_block_max_triton = h8_block_max_hip
masked_full_scores_triton = masked_full_scores_hip
progressive_scores_triton = progressive_scores_hip
two_pass_scores_triton = two_pass_scores_hip
