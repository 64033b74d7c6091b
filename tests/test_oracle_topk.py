"""Pins the top-K oracle (oracle/topk.py) against brute force and the
reference's tie tests (reference tests/test_metrics.py:6-18)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import topk as T


def test_stable_topk_uses_index_tie_break() -> None:
    assert T.stable_topk(np.array([1.0, 3.0, 3.0, 2.0]), 2).tolist() == [1, 2]


def test_stable_topk_resolves_large_cutoff_tie_by_global_index() -> None:
    assert np.array_equal(T.stable_topk(np.ones(64, dtype=np.float32), 8), np.arange(8))


def test_recall_and_random_normalization() -> None:
    assert T.topk_recall(np.array([1, 2]), np.array([2, 3])) == 0.5
    assert T.normalized_recall_lift(0.5, 2, 4) == 0.0
    assert T.topk_recall(np.array([1]), np.array([], dtype=np.int64)) == 1.0
    assert T.normalized_recall_lift(0.3, 8, 8) == 1.0


@pytest.mark.parametrize("seed", range(20))
def test_stable_topk_equals_brute_force(seed: int) -> None:
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 300))
    k = int(rng.integers(1, n + 1))
    # A coarse grid forces many exact ties, including at the cut-off.
    values = rng.integers(-5, 6, size=n).astype(np.float32) if seed % 2 else rng.normal(size=n)
    assert np.array_equal(T.stable_topk(values, k), T.brute_force_topk(values, k))


def test_signed_zeros_tie() -> None:
    values = np.array([-0.0, 0.0, -0.0, -1.0])
    assert T.stable_topk(values, 2).tolist() == [0, 1]
    assert T.brute_force_topk(values, 2).tolist() == [0, 1]


def test_negative_infinity_ranks_last() -> None:
    values = np.array([-np.inf, 1.0, -np.inf, -5.0])
    assert T.stable_topk(values, 3).tolist() == [1, 3, 0]


def test_rejects_bad_k_and_shape() -> None:
    with pytest.raises(ValueError):
        T.stable_topk(np.ones(3), 0)
    with pytest.raises(ValueError):
        T.stable_topk(np.ones(3), 4)
    with pytest.raises(ValueError):
        T.stable_topk(np.ones((2, 2)), 1)


def test_index_order_and_padding_layouts() -> None:
    values = np.array([0.5, 3.0, 3.0, -1.0, 2.0])
    assert T.topk_index_order(values, 3).tolist() == [1, 2, 4]
    assert T.topk_index_order(values, 3, valid=2).tolist() == [0, 1, -1]
    assert T.topk_sorted_padded(values, 7).tolist() == [1, 2, 4, 0, 3, -1, -1]


def test_kth_gap() -> None:
    assert T.kth_gap([4.0, 2.0, 1.0], 1) == pytest.approx(0.5)
    assert T.kth_gap([4.0, 2.0], 2) == np.inf
