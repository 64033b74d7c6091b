"""CPU restatement of the reference's top-K definition (test oracle).

Reference: metrics.py:9-37.  The k largest values; at the cut-off value the
lower indices win; result ordered by (value desc, index asc).  numpy compares
-0.0 equal to +0.0, so the two zeros tie and fall back to the index.
"""

from __future__ import annotations

import numpy as np


def stable_topk(values, k: int) -> np.ndarray:
    """Reference: metrics.py:9-22 (same validation)."""

    x = np.asarray(values)
    if x.ndim != 1:
        raise ValueError(f"expected a vector, got {x.shape}")
    if not 0 < k <= x.size:
        raise ValueError(f"k={k} is invalid for {x.size} values")
    # k-th largest value via a partial sort, then everything above it plus the
    # lowest-index ties at it.
    kth = np.partition(x, x.size - k)[x.size - k]
    above = np.flatnonzero(x > kth)
    ties = np.flatnonzero(x == kth)[: k - above.size]
    chosen = np.concatenate((above, ties))
    order = np.lexsort((chosen, -x[chosen]))
    return chosen[order]


def brute_force_topk(values, k: int) -> np.ndarray:
    """Independent definition: full lexicographic sort on (-value, index)."""

    x = np.asarray(values, dtype=np.float64)
    x = np.where(x == 0.0, 0.0, x)  # -0.0 -> +0.0
    return np.lexsort((np.arange(x.size), -x))[:k]


def topk_index_order(values, k: int, valid: int | None = None) -> np.ndarray:
    """The stable top-k set of the first `valid` values, in ascending index
    order, padded with -1 to k entries (the GPU kernel's unsorted layout)."""

    x = np.asarray(values)
    n = x.size if valid is None else min(valid, x.size)
    if n <= k:
        chosen = np.arange(n)
    else:
        chosen = np.sort(stable_topk(x[:n], k))
    out = np.full(k, -1, dtype=np.int64)
    out[: chosen.size] = chosen
    return out


def topk_sorted_padded(values, k: int, valid: int | None = None) -> np.ndarray:
    """stable_topk of the first `valid` values, padded with -1 to k entries."""

    x = np.asarray(values)
    n = x.size if valid is None else min(valid, x.size)
    out = np.full(k, -1, dtype=np.int64)
    if n == 0:
        return out
    chosen = stable_topk(x[:n], min(k, n))
    out[: chosen.size] = chosen
    return out


def topk_recall(predicted, target) -> float:
    """Reference: metrics.py:25-30."""

    predicted = np.asarray(predicted)
    target = np.asarray(target)
    if target.size == 0:
        return 1.0
    return float(np.intersect1d(predicted, target).size / target.size)


def normalized_recall_lift(recall: float, k: int, length: int) -> float:
    """Reference: metrics.py:33-37."""

    baseline = min(1.0, k / length)
    if baseline == 1.0:
        return 1.0
    return float((recall - baseline) / (1.0 - baseline))


def kth_gap(values, k: int) -> float:
    """Relative gap between the k-th and (k+1)-th largest values (inf if k >= size)."""

    x = np.sort(np.asarray(values, dtype=np.float64))[::-1]
    if k >= x.size:
        return np.inf
    a, b = x[k - 1], x[k]
    return float(abs(a - b) / max(abs(a), abs(b), 1e-30))
