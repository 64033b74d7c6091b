"""The statistics tables of the replay analysis on the GPU (dsa_amd.replay
temporal_stats / block_temporal_stats, reference replay.py:403-474) against
the oracle (oracle/replay.py temporal_stats_rows / block_temporal_stats_rows,
itself pinned to scipy and hand cases in test_oracle_replay_stats.py).

Integer-valued fields and fractions (steps, lengths, k, block sizes, top-k
overlaps, thresholds, cold fractions) and the percentiles (numpy's
arithmetic in the row's precision, over an exact GPU sort) must be equal.
The correlations and the mean block drift are float64 sums in another order
on each side and must agree to 1e-9 relative.  The drift's mean and std: the
reference (and so the oracle) takes numpy's float32 mean and std of the
float32 difference, the kernel sums in float64, so they agree to 1e-5
relative.  Traces: float16 rows (as recorded traces store them, so ties are
common) growing by one key per step, a row with a constant run, and a k the
first transitions cannot hold.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from dsa_amd import replay
from dsa_amd.trace import ScoreTrace
from oracle import replay as R

pytestmark = pytest.mark.gpu


def _trace(seed: int, steps: int, start: int) -> ScoreTrace:
    rng = np.random.default_rng(seed)
    lengths = np.arange(start, start + steps)
    scores = np.full((steps, lengths[-1]), -np.inf, dtype=np.float16)
    base = rng.standard_normal(lengths[-1])
    for t in range(steps):
        row = 0.9 * base[: lengths[t]] + 0.3 * rng.standard_normal(lengths[t])
        scores[t, : lengths[t]] = row.astype(np.float16)
        base = np.concatenate((row, base[lengths[t]:]))
    scores[2, 10:200] = 1.5  # a constant run: many ties in one row
    return ScoreTrace(scores=scores, lengths=lengths, layer=1, workload="synthetic", prompt_id="p0", metadata={})


def _rows(trace: ScoreTrace) -> list[np.ndarray]:
    return [trace.row(t) for t in range(trace.scores.shape[0])]


EXACT_T = ("step", "layer", "context_length", "k", "topk_overlap", "delta_p99_abs")
CLOSE_T = ("score_pearson", "score_spearman")
LOOSE_T = ("delta_mean", "delta_std")
EXACT_B = ("step", "context_length", "k", "block_size", "topk_threshold", "cold_fraction_1", "cold_fraction_2",
           "cold_fraction_4", "cold_fraction_8", "delta_max_p5", "delta_max_median", "delta_max_p95")
CLOSE_B = ("delta_max_mean",)


def _close(a, b, rtol) -> bool:
    if isinstance(b, float) and math.isnan(b):
        return math.isnan(a)
    return abs(a - b) <= rtol * max(1.0, abs(b))


@pytest.mark.parametrize("seed,steps,start", [(1, 6, 700), (2, 4, 4099)])
def test_temporal_stats_match_oracle(device, seed, steps, start) -> None:
    print(f"replay stats: temporal seed={seed} steps={steps} start={start}", flush=True)
    trace = _trace(seed, steps, start)
    got = replay.temporal_stats(trace, [64, 701, 2048]).to_dict("records")
    want = R.temporal_stats_rows(_rows(trace), [64, 701, 2048], layer=1, workload="synthetic", prompt_id="p0")
    assert len(got) == len(want)
    for g, w in zip(got, want):
        for f in EXACT_T:
            assert g[f] == w[f], (f, g, w)
        for f in CLOSE_T:
            assert _close(g[f], w[f], 1e-9), (f, g[f], w[f])
        for f in LOOSE_T:
            assert _close(g[f], w[f], 1e-5), (f, g[f], w[f])


@pytest.mark.parametrize("seed,steps,start", [(3, 7, 300), (4, 4, 4100)])
def test_block_stats_match_oracle(device, seed, steps, start) -> None:
    print(f"replay stats: blocks seed={seed} steps={steps} start={start}", flush=True)
    trace = _trace(seed, steps, start)
    got = replay.block_temporal_stats(trace, [16, 64], [8, 301]).to_dict("records")
    want = R.block_temporal_stats_rows(_rows(trace), [16, 64], [8, 301], layer=1, workload="synthetic",
                                       prompt_id="p0")
    assert len(got) == len(want)
    for g, w in zip(got, want):
        for f in EXACT_B:
            assert g[f] == w[f], (f, g, w)
        for f in CLOSE_B:
            assert _close(g[f], w[f], 1e-9), (f, g[f], w[f])


def test_analyze_writes_the_tables(device, tmp_path) -> None:
    print("replay stats: analyze command", flush=True)
    import argparse

    from dsa_amd import cli
    from dsa_amd.trace import save_trace

    save_trace(tmp_path / "t.npz", _trace(5, 3, 400))
    config = tmp_path / "config.yaml"
    config.write_text("replay:\n  k_values: [64]\n  block_sizes: [16]\n  gamma_sigma: [0.0]\n")
    args = argparse.Namespace(config=config, margin_file=None, trace_roots=[tmp_path], output=tmp_path / "out",
                              wave=1)
    cli.analyze(args)
    import pandas as pd

    t = pd.read_csv(tmp_path / "out" / "temporal_stats.csv")
    b = pd.read_csv(tmp_path / "out" / "block_stats.csv")
    assert list(t.columns) == ["step", "layer", "workload", "prompt_id", "context_length", "score_pearson",
                               "score_spearman", "delta_mean", "delta_std", "delta_p99_abs", "k", "topk_overlap"]
    assert list(b.columns)[:8] == ["step", "layer", "workload", "prompt_id", "context_length", "k", "block_size",
                                   "topk_threshold"]
    assert len(t) > 0 and len(b) > 0
