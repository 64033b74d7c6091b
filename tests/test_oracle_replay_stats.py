"""The oracle's statistics tables (oracle/replay.py temporal_stats_rows /
block_temporal_stats_rows, reference replay.py:403-474) pinned against
independent definitions: scipy's Pearson and Spearman correlations, a
percentile by explicit sorting and linear interpolation, a brute-force
top-k overlap, and a hand-built trace whose cold streaks are known."""

from __future__ import annotations

import math

import numpy as np
import scipy.stats as ss

from oracle import replay as R
from oracle import topk as T


def _percentile(x, q) -> float:
    s = np.sort(np.asarray(x, dtype=np.float64))
    h = (s.size - 1) * q / 100.0
    lo = int(math.floor(h))
    hi = min(lo + 1, s.size - 1)
    return float(s[lo] + (s[hi] - s[lo]) * (h - lo))


def test_correlations_match_scipy() -> None:
    rng = np.random.default_rng(3)
    x = rng.standard_normal(2000).astype(np.float32)
    y = (0.8 * x + 0.3 * rng.standard_normal(2000)).astype(np.float32)
    assert abs(R.pearson(x, y) - ss.pearsonr(x.astype(np.float64), y.astype(np.float64))[0]) < 1e-12
    ties = np.round(x * 2) / 2  # heavy ties: average ranks matter
    assert abs(R.spearman(ties, y) - ss.spearmanr(ties, y)[0]) < 1e-12
    np.testing.assert_array_equal(R.average_ranks(np.array([3.0, 1.0, 3.0, 2.0, -0.0, 0.0])),
                                  [4.5, 2.0, 4.5, 3.0, 0.5, 0.5])
    assert math.isnan(R.pearson(np.ones(5), np.arange(5.0)))
    assert math.isnan(R.pearson([1.0], [2.0]))


def test_temporal_stats_rows_against_direct_formulas() -> None:
    rng = np.random.default_rng(5)
    rows = [rng.standard_normal(300 + t).astype(np.float32) for t in range(4)]
    got = R.temporal_stats_rows(rows, [16, 64, 400], layer=2, workload="w", prompt_id="p")
    assert [(r["step"], r["k"]) for r in got] == [(s, k) for s in (1, 2, 3) for k in (16, 64)]
    for r in got:
        prev, cur = rows[r["step"] - 1], rows[r["step"]]
        n = prev.size
        d = cur[:n] - prev[:n]
        assert r["context_length"] == cur.size
        assert abs(r["delta_mean"] - np.mean(d.astype(np.float64))) < 1e-6
        assert abs(r["delta_std"] - np.std(d.astype(np.float64))) < 1e-6
        assert abs(r["delta_p99_abs"] - _percentile(np.abs(d), 99)) < 1e-6
        a = set(T.brute_force_topk(prev[:n], r["k"]).tolist())
        b = T.brute_force_topk(cur[:n], r["k"])
        assert r["topk_overlap"] == sum(i in a for i in b.tolist()) / r["k"]
        assert abs(r["score_spearman"] - ss.spearmanr(prev[:n], cur[:n])[0]) < 1e-12


def test_block_stats_hand_trace() -> None:
    # Two blocks of 2 keys.  The current k=1 threshold is the row maximum; the
    # block holding it is warm, the other is cold, and streaks count the
    # consecutive cold steps of each block.
    rows = [np.array(v, dtype=np.float32) for v in
            ([0, 1, 2, 3], [9, 1, 2, 3], [0, 1, 2, 8], [0, 1, 2, 8], [7, 1, 2, 3])]
    got = R.block_temporal_stats_rows(rows, [2], [1])
    # cold blocks per step: 1: block 1 (max 3 < 9); 2: block 0; 3: block 0; 4: block 1
    streaks = [(0, 1), (1, 0), (2, 0), (0, 1)]
    for r, (s0, s1) in zip(got, streaks):
        s = np.array([s0, s1])
        assert r["topk_threshold"] == rows[r["step"]].max()
        assert r["cold_fraction_1"] == np.mean(s >= 1)
        assert r["cold_fraction_2"] == np.mean(s >= 2)
        assert r["cold_fraction_4"] == 0.0
    deltas = [np.array([8.0, 0.0]), np.array([-8.0, 5.0]), np.array([0.0, 0.0]), np.array([6.0, -5.0])]
    for r, d in zip(got, deltas):
        assert r["delta_max_mean"] == d.mean()
        assert r["delta_max_p5"] == _percentile(d, 5)
        assert r["delta_max_median"] == _percentile(d, 50)
        assert r["delta_max_p95"] == _percentile(d, 95)


def test_block_stats_growing_rows_and_skipped_k() -> None:
    rng = np.random.default_rng(9)
    rows = [rng.standard_normal(100 + 7 * t).astype(np.float32) for t in range(5)]
    got = R.block_temporal_stats_rows(rows, [16, 32], [8, 120])
    # k = 120 is skipped until the common length reaches it
    ks = [(r["step"], r["block_size"], r["k"]) for r in got]
    assert (3, 16, 120) not in ks and (4, 16, 120) in ks
    for r in got:
        prev, cur = rows[r["step"] - 1], rows[r["step"]]
        n = min(prev.size, cur.size)
        assert r["topk_threshold"] == float(np.partition(cur[:n], -r["k"])[-r["k"]])
        cm, pm = R.block_maxima(cur[:n], r["block_size"]), R.block_maxima(prev[:n], r["block_size"])
        assert abs(r["delta_max_p95"] - _percentile(cm - pm, 95)) < 1e-12
