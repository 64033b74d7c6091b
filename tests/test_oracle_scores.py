"""Pins the CPU score oracle (oracle/scores.py) before it is trusted.

Each check is chosen so that a plausible slip (a dropped ReLU, a sign, a
transposed operand, a wrong head subset) fails: explicit per-key loops on tiny
inputs, hand-computed closed forms, and the reference's own invariants
(tests/test_progressive_kernel.py:31-123 in the reference).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import scores as S


def cpu_inputs(length: int = 129):
    generator = torch.Generator().manual_seed(1582)
    queries = torch.randn(S.HEADS, S.HEAD_DIM, generator=generator)
    weights = torch.randn(S.HEADS, generator=generator)
    keys = torch.randn(length, S.HEAD_DIM, generator=generator)
    return queries, weights, keys


def explicit_scores(q, w, keys) -> np.ndarray:
    """Independent per-key, per-head double loop."""

    q = np.asarray(q, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    out = np.zeros(keys.shape[0])
    for s in range(keys.shape[0]):
        total = 0.0
        for h in range(q.shape[0]):
            dot = float(np.dot(q[h], keys[s]))
            total += w[h] * (dot if dot > 0 else 0.0)
        out[s] = total
    return out


def test_relu_index_score_matches_explicit_loop() -> None:
    q, w, k = cpu_inputs(17)
    np.testing.assert_allclose(S.relu_index_score(q.numpy(), k.numpy(), w.numpy()), explicit_scores(q, w, k), rtol=1e-12, atol=1e-12)


def test_relu_index_score_hand_case() -> None:
    # Two heads, 2-d keys: head 0 sees +3 (kept), head 1 sees -2 (clipped).
    q = np.array([[1.0, 1.0], [-1.0, 0.0]])
    w = np.array([2.0, 5.0])
    keys = np.array([[1.0, 2.0], [-1.0, -1.0]])
    # key 0: dots (3, -1) -> 2*3 + 5*0 = 6; key 1: dots (-2, 1) -> 0 + 5*1 = 5
    np.testing.assert_array_equal(S.relu_index_score(q, keys, w), [6.0, 5.0])


def test_torch_full_scores_matches_explicit_sum() -> None:
    # reference tests/test_progressive_kernel.py:61-67
    q, w, k = cpu_inputs(17)
    torch.testing.assert_close(S.torch_full_scores(q, w, k), torch.from_numpy(explicit_scores(q, w, k)).float(), rtol=1e-5, atol=1e-4)


def test_torch_full_scores_rejects_bad_shapes() -> None:
    q, w, k = cpu_inputs(4)
    with pytest.raises(ValueError):
        S.torch_full_scores(q[:8], w, k)
    with pytest.raises(ValueError):
        S.torch_full_scores(q, w, k[:, :64])


def test_split_head_ids_returns_complement() -> None:
    selected, remaining = S.split_head_ids(torch.tensor([0, 2, 4, 6, 8, 10, 12, 63]))
    assert selected.numel() == 8 and remaining.numel() == 56
    assert sorted(selected.tolist() + remaining.tolist()) == list(range(64))
    assert remaining.tolist() == sorted(remaining.tolist())


@pytest.mark.parametrize("values", [[0, 1], [0, 1, 2, 3, 4, 5, 6, 64], [0, 1, 2, 3, 4, 5, 6, 6]])
def test_split_head_ids_rejects_invalid(values) -> None:
    with pytest.raises(ValueError):
        S.split_head_ids(torch.tensor(values))


def test_dynamic_head_ids_is_stable_for_ties() -> None:
    # reference tests/test_progressive_kernel.py:52-58
    weights = torch.zeros(64)
    weights[20] = -4
    weights[3] = 4
    result = S.dynamic_head_ids(weights)
    assert result.tolist() == [3, 20, 0, 1, 2, 4, 5, 6]


def test_dynamic_head_indices_matches_stable_argsort() -> None:
    gen = torch.Generator().manual_seed(3)
    w = torch.randn(5, 64, generator=gen)
    w[:, 10] = w[:, 11]  # forced ties
    for strategy, key in (("high_weight", w.abs()), ("positive_weight", torch.clamp_min(w, 0))):
        expected = torch.argsort(key, dim=-1, descending=True, stable=True)[:, :8]
        assert torch.equal(S.dynamic_head_indices(w, 8, strategy), expected)


def test_progressive_qk_reduction_closed_forms() -> None:
    # reference tests/test_progressive_kernel.py:103-123
    assert S.progressive_qk_reduction(8192, 0, 0) == pytest.approx(0.875)
    assert S.progressive_qk_reduction(8192, 128, 0) == pytest.approx(0.0)
    expected_work = 2048 * 64 + 6144 * 8 + 1024 * 56
    assert S.progressive_qk_reduction(8192, 32, 16) == pytest.approx(1 - expected_work / (8192 * 64))
    with pytest.raises(ValueError):
        S.progressive_qk_reduction(8192, 129, 0)
    with pytest.raises(ValueError):
        S.progressive_qk_reduction(8192, -1, 0)


def test_progressive_reference_all_promoted_equals_full() -> None:
    # reference tests/test_progressive_kernel.py:70-77
    q, w, k = cpu_inputs(129)
    direct = torch.zeros(math.ceil(len(k) / 64), dtype=torch.bool)
    out, accepted, _ = S.torch_progressive_scores(q, w, k, S.dynamic_head_ids(w), direct, -math.inf)
    torch.testing.assert_close(out, S.torch_full_scores(q, w, k), rtol=1e-5, atol=1e-4)
    assert accepted.all()


def test_progressive_reference_rejects_cold_blocks() -> None:
    # reference tests/test_progressive_kernel.py:80-89
    q, w, k = cpu_inputs(128)
    out, accepted, maxima = S.torch_progressive_scores(q, w, k, S.dynamic_head_ids(w), torch.tensor([True, False]), math.inf)
    assert accepted.tolist() == [True, False]
    assert torch.isfinite(out[:64]).all() and torch.isneginf(out[64:]).all()
    assert torch.isfinite(maxima).all()


def test_progressive_reference_ragged_last_block() -> None:
    # reference tests/test_progressive_kernel.py:92-100
    q, w, k = cpu_inputs(65)
    out, accepted, _ = S.torch_progressive_scores(q, w, k, torch.arange(8), torch.tensor([False, True]), math.inf)
    assert out.shape == (65,) and accepted.tolist() == [False, True] and torch.isfinite(out[-1])


def test_selected_plus_remaining_heads_partition_the_score() -> None:
    q, w, k = cpu_inputs(40)
    sel, rem = S.split_head_ids(torch.tensor([5, 1, 60, 33, 7, 8, 9, 2]))
    part = S._head_subset_scores(q.double().numpy(), w.double().numpy(), k.double().numpy(), sel.numpy())
    rest = S._head_subset_scores(q.double().numpy(), w.double().numpy(), k.double().numpy(), rem.numpy())
    np.testing.assert_allclose(part + rest, explicit_scores(q, w, k), rtol=1e-12, atol=1e-10)
    # and the subset alone is the explicit loop restricted to those heads
    np.testing.assert_allclose(part, explicit_scores(q[sel.long()], w[sel.long()], k), rtol=1e-12, atol=1e-10)


def test_kernel_progressive_semantics() -> None:
    q, w, k = cpu_inputs(200)
    sel, rem = S.split_head_ids(torch.arange(8))
    direct = np.array([1, 0, 0, 1], dtype=bool)
    part, maxima = S.kernel_h8_block_max(q.numpy(), w.numpy(), k.numpy(), sel.numpy(), ~direct, 64)
    threshold = float(np.median(maxima[1:3]))
    out, accepted, block_max = S.kernel_progressive(q.numpy(), w.numpy(), k.numpy(), sel.numpy(), rem.numpy(), direct, threshold, 64)
    full = explicit_scores(q, w, k)
    assert np.isneginf(block_max[direct]).all()
    np.testing.assert_allclose(block_max[~direct], maxima[~direct])
    assert accepted.tolist() == [True, *(maxima[1:3] >= threshold).tolist(), True]
    for b in range(4):
        lo, hi = 64 * b, min(200, 64 * (b + 1))
        if accepted[b]:
            np.testing.assert_allclose(out[lo:hi], full[lo:hi], rtol=1e-10, atol=1e-9)
        else:
            assert np.isneginf(out[lo:hi]).all()
    masked = S.kernel_masked_full(q.numpy(), w.numpy(), k.numpy(), accepted, 64)
    np.testing.assert_array_equal(np.isneginf(masked), np.isneginf(out))


def test_score_encoded_and_causal_mask() -> None:
    gen = torch.Generator().manual_seed(7)
    q = torch.randn(2, 3, 64, 128, generator=gen)
    w = torch.randn(2, 3, 64, generator=gen)
    k = torch.randn(2, 5, 128, generator=gen)
    dense = S.score_encoded(q.numpy(), w.numpy(), k.numpy())
    for b in range(2):
        for t in range(3):
            np.testing.assert_allclose(dense[b, t], explicit_scores(q[b, t], w[b, t], k[b]), rtol=1e-12, atol=1e-10)
    causal = S.score_encoded(q.numpy(), w.numpy(), k.numpy(), causal_offset=2)
    for t in range(3):
        np.testing.assert_array_equal(causal[:, t, : t + 3], dense[:, t, : t + 3])
        assert np.isneginf(causal[:, t, t + 3 :]).all()


def test_score_head_sparse_fixed_and_dynamic() -> None:
    gen = torch.Generator().manual_seed(8)
    q = torch.randn(3, 64, 128, generator=gen)
    w = torch.randn(3, 64, generator=gen)
    k = torch.randn(9, 128, generator=gen)
    fixed = S.score_head_sparse(q.numpy(), w.numpy(), k.numpy(), [4, 0, 9])
    for t in range(3):
        np.testing.assert_allclose(fixed[t], explicit_scores(q[t, [4, 0, 9]], w[t, [4, 0, 9]], k), rtol=1e-12, atol=1e-10)
    ids = np.array([[1, 2], [3, 4], [63, 0]])
    dyn = S.score_head_sparse(q.numpy(), w.numpy(), k.numpy(), ids)
    for t in range(3):
        np.testing.assert_allclose(dyn[t], explicit_scores(q[t, ids[t]], w[t, ids[t]], k), rtol=1e-12, atol=1e-10)


def test_fp8_dequantization_is_scale_times_value() -> None:
    values = torch.tensor([[0.5, -1.0] + [0.0] * 126] * 130, dtype=torch.float32).to(torch.float8_e4m3fn)
    scales = torch.tensor([2.0, 3.0])
    deq = S.dequantize_fp8_blocks(values, scales)
    assert deq.shape == (130, 128)
    assert deq[0, 0] == 1.0 and deq[127, 1] == -2.0 and deq[128, 0] == 1.5 and deq[129, 1] == -3.0
