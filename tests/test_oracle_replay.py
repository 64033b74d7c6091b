"""Pins the temporal replay oracle (oracle/replay.py).

Reference replay tests (reference tests/test_replay.py:6-57), hand-built cases
with counts worked out on paper, invariants (full scores everything, oracle is
exact, a huge margin is exact, wave=1 is the reference schedule, a single wave
decides everything against the seed threshold), and
an independent key-by-key simulator of the compiled reference path
(reference replay.py:47-109, heap-based threshold).
"""

from __future__ import annotations

import heapq
import math

import numpy as np
import pytest

from oracle import replay as R
from oracle.topk import stable_topk


def test_large_margin_replay_is_exact() -> None:
    rng = np.random.default_rng(4)
    previous = rng.normal(size=512)
    current = np.concatenate([previous + 0.001 * rng.normal(size=512), [0.0]])
    result = R.replay_transition(previous, current, k=32, block_size=16, gamma_sigma=10.0, method="dynamic", scan_order="previous_hot")
    assert result.exact_match and result.recall == 1.0 and 0 <= result.qk_reduction <= 1


def test_oracle_is_exact_and_never_scores_more_than_full() -> None:
    rng = np.random.default_rng(5)
    previous = rng.normal(size=257)
    current = np.concatenate([rng.normal(size=257), [3.0]])
    result = R.replay_transition(previous, current, k=16, block_size=32, gamma_sigma=0.0, method="oracle", scan_order="oracle_current")
    assert result.exact_match and result.qk_scored <= current.size


def test_empirical_zero_margin_reports_miss() -> None:
    previous = np.zeros(64)
    previous[:4] = 2.0
    current = previous.copy()
    current[40:44] = 3.0
    result = R.replay_transition(previous, current, k=4, block_size=8, gamma_sigma=0.0, method="dynamic", scan_order="previous_hot")
    assert not result.exact_match and result.false_cold_blocks > 0


def test_hand_case_counts() -> None:
    # 4 blocks of 4 keys.  previous top-2 = keys 0, 1 (block 0).
    previous = np.array([9, 8, 0, 0, 1, 1, 1, 1, 5, 0, 0, 0, 0, 0, 0, 0], dtype=float)
    current = previous.copy()
    current[9] = 8.5  # a new top-2 key in block 2 (previous max 5)
    # block maxima prev: [9, 1, 5, 0]; gamma = 0; seed = {0, 1}; tau_seed = 8.
    static = R.replay_transition(previous, current, k=2, block_size=4, gamma_sigma=0.0, method="static")
    # static keeps only blocks with upper >= 8: block 0 -> scores keys 2, 3 (seeds excluded)
    assert static.qk_scored == 2 + 2
    assert static.blocks_pruned == 3
    assert static.false_cold_blocks == 1  # block 2 holds key 9 (score 8.5, rank 2)
    assert static.recall == 0.5 and not static.exact_match
    assert static.tau_seed == 8.0 and static.tau_final == 8.5
    assert static.threshold_gap == pytest.approx(0.5)
    assert static.discovery_fraction == 1.0  # a true key was never evaluated
    # full: everything
    full = R.replay_transition(previous, current, k=2, block_size=4, gamma_sigma=0.0, method="full")
    assert full.qk_scored == 16 and full.exact_match and full.discovery_fraction == 1.0
    # bytes: metadata 4 blocks * 8 B, keys 256 B each
    assert static.metadata_bytes == 32
    assert static.net_byte_reduction == pytest.approx(1 - (4 * 256 + 32) / (16 * 256))


def test_new_tail_block_is_never_pruned() -> None:
    previous = np.array([5.0, 4.0, 0.0, 0.0, 0.0, 0.0])
    current = np.array([5.0, 4.0, 0.0, 0.0, 0.0, 0.0, 9.0])
    # blocks of 4: block 1 holds keys 4..6 and key 6 is new -> upper = +inf
    result = R.replay_transition(previous, current, k=2, block_size=4, gamma_sigma=0.0, method="static")
    assert result.exact_match and result.blocks_pruned == 0


def test_scan_orders() -> None:
    upper = np.array([1.0, 3.0, 3.0, 2.0])
    current_max = np.array([0.0, 5.0, 1.0, 5.0])
    hot = np.array([False, False, True, True])
    assert R.block_scan_order("address", upper, current_max, hot).tolist() == [0, 1, 2, 3]
    assert R.block_scan_order("previous_hot", upper, current_max, hot).tolist() == [2, 3, 1, 0]
    assert R.block_scan_order("upper_hot", upper, current_max, hot).tolist() == [1, 2, 3, 0]
    assert R.block_scan_order("oracle_current", upper, current_max, hot).tolist() == [1, 3, 2, 0]
    with pytest.raises(ValueError):
        R.block_scan_order("bogus", upper, current_max, hot)


def heap_simulator(current, seed, truth, upper, order, block_size, fixed, dynamic):
    """Key-by-key restatement of the compiled reference path (replay.py:47-109)."""

    length = current.size
    k = truth.size
    seeded = np.zeros(length, bool)
    in_truth = np.zeros(length, bool)
    in_truth[truth] = True
    truth_block = np.zeros(upper.size, bool)
    truth_block[truth // block_size] = True
    heap = []
    scored = true_seen = last = 0
    for key in seed:
        seeded[key] = True
        heapq.heappush(heap, (current[key], -key))
        scored += 1
        if in_truth[key]:
            true_seen += 1
            last = scored
    threshold = heap[0][0] if dynamic else fixed
    pruned = false_cold = 0
    for b in order:
        if upper[b] < threshold:
            pruned += 1
            false_cold += truth_block[b]
            continue
        for key in range(b * block_size, min(length, (b + 1) * block_size)):
            if seeded[key]:
                continue
            scored += 1
            if in_truth[key]:
                true_seen += 1
                last = scored
            if dynamic and (current[key], -key) > heap[0]:
                heapq.heapreplace(heap, (current[key], -key))
                threshold = heap[0][0]
    discovery = 1.0 if true_seen < k else last / length
    return scored, pruned, false_cold, true_seen, discovery


@pytest.mark.parametrize("seed", range(12))
def test_matches_key_by_key_simulator(seed: int) -> None:
    rng = np.random.default_rng(100 + seed)
    n_prev = int(rng.integers(64, 400))
    grow = int(rng.integers(0, 3))
    previous = rng.normal(size=n_prev)
    current = np.concatenate([previous + rng.normal(scale=0.3, size=n_prev), rng.normal(size=grow)])
    if seed % 3 == 0:
        current = np.round(current * 4) / 4  # ties
    k = int(rng.integers(1, min(40, n_prev)))
    bs = int(rng.choice([4, 8, 16, 32]))
    gs = float(rng.choice([0.0, 0.25, 1.0]))
    for method, order_name in [("static", "address"), ("static_hot_first", "previous_hot"), ("dynamic", "address"), ("dynamic", "previous_hot"), ("dynamic", "upper_hot"), ("oracle", "oracle_current")]:
        res = R.replay_transition(previous, current, k=k, block_size=bs, gamma_sigma=gs, method=method, scan_order=order_name)
        cur_max, prev_max, sigma = R.transition_setup(previous, current, bs)
        upper = R.upper_bounds(prev_max, gs * sigma, previous.size, current.size, bs)
        seed_ids = stable_topk(previous, k)
        truth = stable_topk(current, k)
        order_used, dynamic, oracle_bound = R.method_schedule(method, order_name)
        bound = cur_max if oracle_bound else upper
        hot = np.zeros(bound.size, bool)
        hot[seed_ids // bs] = True
        order = R.block_scan_order(order_used, bound, cur_max, hot)
        sim = heap_simulator(current, seed_ids, truth, bound, order, bs, float(np.min(current[seed_ids])), dynamic)
        assert (res.qk_scored, res.blocks_pruned, res.false_cold_blocks) == sim[:3], (method, order_name)
        assert res.recall == sim[3] / k
        assert res.discovery_fraction == pytest.approx(sim[4])


def test_wave_one_is_reference_and_one_wave_is_static() -> None:
    rng = np.random.default_rng(9)
    previous = rng.normal(size=2048)
    current = previous + 0.2 * rng.normal(size=2048)
    ref = R.replay_transition(previous, current, k=64, block_size=16, gamma_sigma=0.5, method="dynamic", scan_order="previous_hot")
    w1 = R.replay_transition(previous, current, k=64, block_size=16, gamma_sigma=0.5, method="dynamic", scan_order="previous_hot", wave=1)
    assert ref == w1
    # One wave holding every block decides everything against tau_seed: the
    # dynamic schedule then equals the static one with the same order.
    blocks = math.ceil(2048 / 16)
    one_wave = R.replay_transition(previous, current, k=64, block_size=16, gamma_sigma=0.5, method="dynamic", scan_order="previous_hot", wave=blocks)
    static_hot = R.replay_transition(previous, current, k=64, block_size=16, gamma_sigma=0.5, method="static_hot_first")
    assert (one_wave.qk_scored, one_wave.blocks_pruned, one_wave.recall) == (static_hot.qk_scored, static_hot.blocks_pruned, static_hot.recall)
    # static thresholds never change, so waves do not matter
    s1 = R.replay_transition(previous, current, k=64, block_size=16, gamma_sigma=0.5, method="static")
    s9 = R.replay_transition(previous, current, k=64, block_size=16, gamma_sigma=0.5, method="static", wave=9)
    assert s1 == s9


def test_replay_trace_rows_and_aggregate() -> None:
    rng = np.random.default_rng(11)
    rows = [rng.normal(size=100)]
    for _ in range(3):
        rows.append(np.concatenate([rows[-1] + 0.1 * rng.normal(size=rows[-1].size), rng.normal(size=1)]))
    out = R.replay_trace_rows(rows, k_values=[8, 1000], block_sizes=[16, 32], gamma_sigma_values=[0.0, 1.0], absolute_margins={16: 0.5})
    # per (step, k=8, bs): 2 invariant + 2*6 sweep (+5 calibrated at bs 16)
    assert len(out) == 3 * ((2 + 12 + 5) + (2 + 12))
    agg = R.aggregate_rows(out)
    assert set(agg["method"]) == {"full", "oracle", "static", "static_hot_first", "dynamic"}
    assert (agg["transition_count"] == 3).all()
    full = agg[agg["method"] == "full"]
    assert (full["qk_reduction"] == 0).all() and (full["exact_match"] == 1.0).all()


def test_rejects_bad_inputs() -> None:
    with pytest.raises(ValueError):
        R.replay_transition(np.zeros(5), np.zeros(4), k=1, block_size=2, gamma_sigma=0, method="full")
    with pytest.raises(ValueError):
        R.replay_transition(np.zeros(5), np.zeros(5), k=6, block_size=2, gamma_sigma=0, method="full")
    with pytest.raises(ValueError):
        R.replay_transition(np.zeros(5), np.zeros(5), k=1, block_size=2, gamma_sigma=0, method="bogus")
