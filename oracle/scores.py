"""CPU restatement of the indexer score functions (test oracle).

score_s = sum_h w_h * max(0, q_h . k_s) with 64 heads x 128 dims.
"""

from __future__ import annotations

import math

import numpy as np
import torch

HEADS = 64
HEAD_DIM = 128
VERIFIER_HEADS = 8


def relu_index_score(q, keys, weights) -> np.ndarray:
    """Float64 score of every key.  Reference: certified.py:6-15."""

    q = np.asarray(q, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    weights = np.asarray(weights, dtype=np.float64)
    if q.ndim != 2 or keys.ndim != 2 or q.shape[1] != keys.shape[1]:
        raise ValueError("q must be [heads,dim] and keys [tokens,dim]")
    if weights.shape != (q.shape[0],):
        raise ValueError("weights must have one value per head")
    dots = keys @ q.T  # [tokens, heads]
    return np.maximum(dots, 0.0) @ weights


def abs_weight_scale(q, keys, weights) -> np.ndarray:
    """sum_h |w_h| max(0, q_h.k): the magnitude used for relative tolerances."""

    return relu_index_score(q, keys, np.abs(np.asarray(weights, dtype=np.float64)))


def torch_full_scores(queries: torch.Tensor, weights: torch.Tensor, keys: torch.Tensor) -> torch.Tensor:
    """fp32 dense score.  Reference: progressive_kernel.py:45-55."""

    if queries.shape != (HEADS, HEAD_DIM) or weights.shape != (HEADS,):
        raise ValueError("expected queries [64,128] and weights [64]")
    if keys.ndim != 2 or keys.shape[1] != HEAD_DIM:
        raise ValueError("expected keys [L,128]")
    head_dots = queries.float() @ keys.float().T  # [64, L]
    return torch.einsum("hl,h->l", torch.clamp_min(head_dots, 0.0), weights.float())


def split_head_ids(selected) -> tuple[torch.Tensor, torch.Tensor]:
    """Reference: progressive_kernel.py:23-34."""

    ids = torch.as_tensor(selected, dtype=torch.int32).cpu()
    if ids.ndim != 1 or ids.numel() != VERIFIER_HEADS:
        raise ValueError("selected head IDs must have shape [8]")
    if int(ids.min()) < 0 or int(ids.max()) >= HEADS:
        raise ValueError("head ID outside [0, 64)")
    if len(set(ids.tolist())) != VERIFIER_HEADS:
        raise ValueError("selected head IDs must be unique")
    chosen = set(ids.tolist())
    rest = torch.tensor([h for h in range(HEADS) if h not in chosen], dtype=torch.int32)
    return ids.contiguous(), rest


def dynamic_head_ids(weights: torch.Tensor, width: int = VERIFIER_HEADS) -> torch.Tensor:
    """Top-|w| head ids, lower id first on ties.  Reference: progressive_kernel.py:37-42."""

    if tuple(weights.shape) != (HEADS,):
        raise ValueError("weights must have shape [64]")
    if not 0 < width <= HEADS:
        raise ValueError("invalid head width")
    magnitude = weights.detach().cpu().abs().tolist()
    order = sorted(range(HEADS), key=lambda h: (-magnitude[h], h))
    return torch.tensor(order[:width], dtype=torch.int32)


def dynamic_head_indices(weights: torch.Tensor, width: int, strategy: str) -> torch.Tensor:
    """Per-row stable top-`width` heads.  Reference: verifier_scoring.py:142-159."""

    w = weights.detach().cpu().float()
    if not 0 < width <= w.shape[-1]:
        raise ValueError("invalid head width")
    if strategy == "high_weight":
        key = w.abs()
    elif strategy == "positive_weight":
        key = torch.clamp_min(w, 0)
    else:
        raise ValueError("strategy must be high_weight or positive_weight")
    rows = []
    for row in key.reshape(-1, key.shape[-1]).tolist():
        rows.append(sorted(range(len(row)), key=lambda h: (-row[h], h))[:width])
    return torch.tensor(rows, dtype=torch.int64)


def progressive_qk_reduction(length: int, direct_full_blocks: int, promoted_cold_blocks: int, *, block_size: int = 64) -> float:
    """Reference: progressive_kernel.py:93-111."""

    blocks = math.ceil(length / block_size)
    if direct_full_blocks < 0 or promoted_cold_blocks < 0:
        raise ValueError("block counts must be non-negative")
    if direct_full_blocks + promoted_cold_blocks > blocks:
        raise ValueError("accepted block counts exceed total blocks")
    direct_tokens = min(length, direct_full_blocks * block_size)
    promoted_tokens = min(length - direct_tokens, promoted_cold_blocks * block_size)
    head_work = (
        direct_tokens * HEADS
        + (length - direct_tokens) * VERIFIER_HEADS
        + promoted_tokens * (HEADS - VERIFIER_HEADS)
    )
    return 1.0 - head_work / (length * HEADS)


def _head_subset_scores(q: np.ndarray, w: np.ndarray, keys: np.ndarray, heads) -> np.ndarray:
    heads = np.asarray(heads, dtype=np.int64)
    dots = keys @ q[heads].T
    return np.maximum(dots, 0.0) @ w[heads]


def torch_progressive_scores(queries, weights, keys, selected_heads, direct_full_blocks, threshold: float, *, block_size: int = 64):
    """Sequential progressive reference.  Reference: progressive_kernel.py:58-90.

    Note the reference CPU semantics: ``block_max`` holds the H8 partial maximum
    for direct blocks as well.  Returns float32 torch tensors like the reference.
    """

    selected, remaining = split_head_ids(torch.as_tensor(selected_heads).cpu())
    q = queries.detach().cpu().double().numpy()
    w = weights.detach().cpu().double().numpy()
    k = keys.detach().cpu().double().numpy()
    length = k.shape[0]
    blocks = math.ceil(length / block_size)
    direct = torch.as_tensor(direct_full_blocks).cpu().bool().numpy()
    if direct.size != blocks:
        raise ValueError("direct_full_blocks length mismatch")
    out = np.full(length, -np.inf)
    accepted = direct.copy()
    block_max = np.full(blocks, -np.inf)
    for b in range(blocks):
        lo, hi = b * block_size, min(length, (b + 1) * block_size)
        partial = _head_subset_scores(q, w, k[lo:hi], selected.numpy())
        block_max[b] = partial.max()
        if accepted[b] or block_max[b] >= threshold:
            accepted[b] = True
            out[lo:hi] = partial + _head_subset_scores(q, w, k[lo:hi], remaining.numpy())
    return (
        torch.from_numpy(out.astype(np.float32)),
        torch.from_numpy(accepted),
        torch.from_numpy(block_max.astype(np.float32)),
    )


def kernel_progressive(q, w, keys, selected, remaining, direct, threshold: float, block_size: int):
    """GPU-kernel semantics of the fused progressive pass (float64).

    Reference: progressive_kernel.py:277-346.  Direct blocks: all 64 heads and
    block_max = -inf.  Other blocks: H8 partial, promote iff max >= threshold.
    Returns (scores with -inf for rejected blocks, accepted bool, block_max).
    """

    q = np.asarray(q, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    length = keys.shape[0]
    blocks = math.ceil(length / block_size)
    direct = np.asarray(direct).astype(bool)
    out = np.full(length, -np.inf)
    accepted = np.zeros(blocks, dtype=bool)
    block_max = np.full(blocks, -np.inf)
    for b in range(blocks):
        lo, hi = b * block_size, min(length, (b + 1) * block_size)
        if direct[b]:
            accepted[b] = True
            out[lo:hi] = relu_index_score(q, keys[lo:hi], w)
            continue
        partial = _head_subset_scores(q, w, keys[lo:hi], selected)
        block_max[b] = partial.max()
        if block_max[b] >= threshold:
            accepted[b] = True
            out[lo:hi] = partial + _head_subset_scores(q, w, keys[lo:hi], remaining)
    return out, accepted, block_max


def kernel_h8_block_max(q, w, keys, selected, cold, block_size: int):
    """GPU-kernel semantics of the H8 pass.  Reference: progressive_kernel.py:218-246."""

    keys = np.asarray(keys, dtype=np.float64)
    length = keys.shape[0]
    blocks = math.ceil(length / block_size)
    cold = np.asarray(cold).astype(bool)
    partial = np.full(length, -np.inf)
    maxima = np.full(blocks, -np.inf)
    for b in range(blocks):
        if not cold[b]:
            continue
        lo, hi = b * block_size, min(length, (b + 1) * block_size)
        partial[lo:hi] = _head_subset_scores(np.asarray(q, np.float64), np.asarray(w, np.float64), keys[lo:hi], selected)
        maxima[b] = partial[lo:hi].max()
    return partial, maxima


def kernel_masked_full(q, w, keys, keep, block_size: int) -> np.ndarray:
    """Reference: progressive_kernel.py:249-274 (full score on kept blocks, -inf else)."""

    keys = np.asarray(keys, dtype=np.float64)
    out = np.full(keys.shape[0], -np.inf)
    keep = np.asarray(keep).astype(bool)
    for b in np.flatnonzero(keep):
        lo, hi = b * block_size, min(keys.shape[0], (b + 1) * block_size)
        out[lo:hi] = relu_index_score(q, keys[lo:hi], w)
    return out


def score_encoded(queries, weights, keys, *, causal_offset: int | None = None) -> np.ndarray:
    """Batched / multi-query scores ``[B,Q,K]`` in float64.

    Reference: sidecar.py:89-107 (without the bf16 rounding of the einsum).
    ``causal_offset`` masks key j of query t unless j <= t + offset (-inf).
    """

    q = np.asarray(queries, dtype=np.float64)
    w = np.asarray(weights, dtype=np.float64)
    k = np.asarray(keys, dtype=np.float64)
    batch, num_queries, _, _ = q.shape
    length = k.shape[1]
    out = np.empty((batch, num_queries, length))
    for b in range(batch):
        for t in range(num_queries):
            out[b, t] = relu_index_score(q[b, t], k[b], w[b, t])
            if causal_offset is not None:
                out[b, t, t + causal_offset + 1 :] = -np.inf
    return out


def score_head_sparse(queries, weights, keys, head_indices) -> np.ndarray:
    """Selected-head scores ``[Q,K]`` in float64.  Reference: verifier_scoring.py:49-92."""

    q = np.asarray(queries, dtype=np.float64)
    w = np.asarray(weights, dtype=np.float64)
    k = np.asarray(keys, dtype=np.float64)
    ids = np.asarray(head_indices, dtype=np.int64)
    out = np.empty((q.shape[0], k.shape[0]))
    for t in range(q.shape[0]):
        row_ids = ids if ids.ndim == 1 else ids[t]
        out[t] = _head_subset_scores(q[t], w[t], k, row_ids)
    return out


def dequantize_fp8_blocks(keys_fp8: torch.Tensor, scales: torch.Tensor) -> np.ndarray:
    """fp8 e4m3fn keys [..., L, 128] times their per-128-key scale -> float64."""

    values = keys_fp8.cpu().float().double().numpy()
    s = scales.cpu().double().numpy()
    repeat = np.repeat(s, 128, axis=-1)[..., : values.shape[-2]]
    return values * repeat[..., None]
