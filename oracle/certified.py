"""CPU restatement of the certified temporal bound (test oracle).

Reference: certified.py:18-62.  Per key block b and head h, with n_bh the
largest key norm in the block, ReLU's 1-Lipschitz property and Cauchy-Schwarz
give |w_t ReLU(q_t.k) - w_p ReLU(q_p.k)| <= (|w_t - w_p| ||q_p|| + |w_t|
||q_t - q_p||) ||k||, summed over heads.
"""

from __future__ import annotations

import numpy as np


def temporal_score_radius(q_now, q_prev, w_now, w_prev, block_key_norm) -> np.ndarray:
    """Reference: certified.py:18-48."""

    q_now = np.asarray(q_now, dtype=np.float64)
    q_prev = np.asarray(q_prev, dtype=np.float64)
    w_now = np.asarray(w_now, dtype=np.float64)
    w_prev = np.asarray(w_prev, dtype=np.float64)
    norms = np.asarray(block_key_norm, dtype=np.float64)
    if q_now.shape != q_prev.shape or q_now.ndim != 2:
        raise ValueError("query tensors must have shape [heads,dim]")
    if w_now.shape != w_prev.shape or w_now.shape != (q_now.shape[0],):
        raise ValueError("weight tensors must have shape [heads]")
    if norms.ndim != 2 or norms.shape[1] != q_now.shape[0]:
        raise ValueError("block_key_norm must have shape [blocks,heads]")
    per_head = np.abs(w_now - w_prev) * np.sqrt((q_prev ** 2).sum(axis=1)) + np.abs(w_now) * np.sqrt(((q_now - q_prev) ** 2).sum(axis=1))
    return norms @ per_head


def block_key_norms(keys, block_size: int) -> np.ndarray:
    """Largest key L2 norm per block and head, keys [tokens, heads, dim].  Reference: certified.py:51-62."""

    keys = np.asarray(keys, dtype=np.float64)
    if keys.ndim != 3:
        raise ValueError("keys must have shape [tokens,heads,dim]")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    norms = np.sqrt((keys ** 2).sum(axis=2))  # [tokens, heads]
    blocks = (keys.shape[0] + block_size - 1) // block_size
    return np.stack([norms[b * block_size : (b + 1) * block_size].max(axis=0) for b in range(blocks)])


SCORE_ROUNDING_ALLOWANCE = 2.0**-15


def certified_margins(q_now, q_prev, w_now, w_prev, keys, block_size: int) -> np.ndarray:
    """Per-block margins of a temporal step over one sequence's shared-key
    cache: ``temporal_score_radius`` (certified.py:18-48) with every head's
    block norm equal to the block's largest key norm, plus the fp32 score
    rounding allowance ``2^-15 * n_b * sum_h (|w_now| ||q_now|| + |w_prev|
    ||q_prev||)`` of the two steps' kernel scores.  q [heads, dim], w [heads],
    keys [tokens, dim] (the previous step's keys)."""

    q_now = np.asarray(q_now, dtype=np.float64)
    q_prev = np.asarray(q_prev, dtype=np.float64)
    w_now = np.asarray(w_now, dtype=np.float64)
    w_prev = np.asarray(w_prev, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    heads = q_now.shape[0]
    block_norm = block_key_norms(keys[:, None, :], block_size)[:, 0]  # [blocks]
    radius = temporal_score_radius(q_now, q_prev, w_now, w_prev, np.repeat(block_norm[:, None], heads, axis=1))
    slack = np.abs(w_now) * np.sqrt((q_now ** 2).sum(axis=1)) + np.abs(w_prev) * np.sqrt((q_prev ** 2).sum(axis=1))
    return radius + SCORE_ROUNDING_ALLOWANCE * block_norm * slack.sum()
