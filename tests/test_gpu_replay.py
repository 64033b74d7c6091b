"""GPU replay over recorded score traces against the reference's own output.

``tests/golden/replay_vectors.json`` holds the per-transition rows and the
aggregate of the reference's ``replay_trace`` (replay.py:476-627) on a seeded
float32 trace (5 steps from 300 keys, K 8 / 32, blocks 16 / 32, gamma_sigma
0 / 0.5, a calibrated margin at block 16), written by the reference itself
(tests/golden/make_replay_vectors.py).  ``dsa_amd.replay`` runs every filter
of that sweep in the HIP temporal kernels with the trace rows as the score
source; every field of every row and of the aggregate must match (floats to
1e-12 relative, integers and flags exactly).  The same holds against the
oracle (oracle/replay.py) on float32 transitions with dynamic refreshes every
wave of 1, 3 and 8 blocks, and collect_trace's rows against the dense kernel.
"""

from __future__ import annotations

import dataclasses
import importlib.util
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from dsa_amd import replay
from dsa_amd.trace import ScoreTrace, collect_trace
from oracle import replay as R
from oracle.scores import relu_index_score

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
_spec = importlib.util.spec_from_file_location("make_replay_vectors", GOLDEN / "make_replay_vectors.py")
gen = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(gen)
RESULTS = json.loads((GOLDEN / "replay_vectors.json").read_text())


def same(expected, got) -> bool:
    if isinstance(expected, str) and expected in ("nan", "inf", "-inf"):
        return math.isnan(got) if expected == "nan" else got == float(expected)
    if isinstance(expected, bool) or isinstance(got, (bool, np.bool_)):
        return bool(expected) == bool(got)
    if isinstance(expected, int):
        return int(got) == expected
    if isinstance(expected, float):
        g = float(got)
        if math.isnan(g):
            return False
        return g == expected or abs(g - expected) <= 1e-12 * max(1.0, abs(expected))
    return expected == got


def golden_trace() -> ScoreTrace:
    scores, lengths = gen.make_score_rows(4242)
    return ScoreTrace(scores=scores, lengths=lengths, layer=3, workload="synthetic", prompt_id="p7", metadata={})


def test_replay_trace_rows_match_reference(device) -> None:
    got = replay.replay_trace_rows(golden_trace(), k_values=gen.TRACE_K, block_sizes=gen.TRACE_BLOCKS,
                                   gamma_sigma_values=gen.TRACE_GAMMAS, absolute_margins=gen.TRACE_MARGINS)
    want = RESULTS["trace_rows"]
    assert len(got) == len(want)
    for g, w in zip(got, want):
        assert set(g) == set(w)
        for field, expected in w.items():
            assert same(expected, g[field]), (w["step"], w["k"], w["block_size"], w["method"], w["scan_order"],
                                              w["gamma_sigma"], field, expected, g[field])


def test_replay_trace_summary_matches_reference(device) -> None:
    summary = replay.replay_trace(golden_trace(), k_values=gen.TRACE_K, block_sizes=gen.TRACE_BLOCKS,
                                  gamma_sigma_values=gen.TRACE_GAMMAS, absolute_margins=gen.TRACE_MARGINS)
    want = RESULTS["trace_summary"]
    got = summary.to_dict("records")
    assert len(got) == len(want)
    for g, w in zip(got, want):
        for field, expected in w.items():
            assert same(expected, g[field]), (w["k"], w["block_size"], w["method"], field, expected, g[field])


@pytest.mark.parametrize("wave", [1, 3, 8])
@pytest.mark.parametrize("method,order", [("static", "address"), ("static_hot_first", "previous_hot"),
                                          ("dynamic", "address"), ("dynamic", "previous_hot"),
                                          ("dynamic", "upper_hot"), ("dynamic", "oracle_current"),
                                          ("oracle", "oracle_current")])
def test_replay_transition_matches_oracle(device, method, order, wave) -> None:
    for t, (lp, lc) in enumerate(gen.TRANSITIONS):
        previous, current = gen.make_transition(1582 + t, lp, lc)
        previous, current = previous.astype(np.float32), current.astype(np.float32)
        for k in (16, 64):
            for bs in (16, 64):
                for gs in (0.0, 0.5):
                    want = dataclasses.asdict(R.replay_transition(
                        previous, current, k=k, block_size=bs, gamma_sigma=gs, method=method, scan_order=order,
                        step=t, wave=wave, sigma=float(np.std(current[: previous.size] - previous))))
                    got = dataclasses.asdict(replay.replay_transition(
                        previous, current, k=k, block_size=bs, gamma_sigma=gs, method=method, scan_order=order,
                        step=t, wave=wave))
                    for field, expected in want.items():
                        g = got[field]
                        ok = (math.isnan(g) and math.isnan(expected)) if isinstance(expected, float) and math.isnan(expected) \
                            else g == expected
                        assert ok, (t, k, bs, gs, field, expected, g)


def test_collect_trace_rows_are_the_dense_scores(device) -> None:
    gen_t = torch.Generator().manual_seed(9)
    keys = torch.randn(700, 128, generator=gen_t).to(torch.bfloat16)
    q = (torch.randn(4, 64, 128, generator=gen_t) / math.sqrt(128)).to(torch.bfloat16)
    w = torch.randn(64, generator=gen_t) / 8
    lengths = np.array([600, 601, 650, 700])
    trace = collect_trace(q.to(device), w.to(device), keys.to(device), lengths, layer=2, prompt_id="x")
    assert trace.scores.dtype == np.float16 and trace.scores.shape == (4, 700)
    for t, n in enumerate(lengths):
        want = relu_index_score(q[t].float().numpy(), keys[:n].float().numpy(), w.numpy())
        row = trace.row(t)
        assert row.size == n
        np.testing.assert_allclose(row, want, rtol=2e-3, atol=2e-3 * np.abs(want).max())
        assert np.all(np.isneginf(trace.scores[t, n:]))


@pytest.mark.parametrize("order", ["previous_hot", "upper_hot", "oracle_current"])
@pytest.mark.parametrize("gamma", [0.05, 1.0e8])
def test_scan_order_matches_oracle(device, order, gamma) -> None:
    # The scan order of the prep kernel against the oracle's sort (replay.py:
    # 153-169).  A margin of 1e8 makes the float64 bounds of distinct block
    # maxima round to one float, so the packed (float-keyed) sort must fall
    # back to the exact float64 order.
    rng = np.random.default_rng(7)
    length, k, bs = 3000, 64, 16
    previous = rng.standard_normal(length - 3).astype(np.float32)
    current = np.concatenate([0.9 * previous + 0.1 * rng.standard_normal(previous.size), rng.standard_normal(3)])
    current = current.astype(np.float32)
    seed = torch.from_numpy(np.argsort(-previous.astype(np.float64), kind="stable")[:k].copy()).to(device)
    truth = torch.from_numpy(np.argsort(-current.astype(np.float64), kind="stable")[:k].copy()).to(device)
    t = replay._Transition(torch.from_numpy(previous).to(device), torch.from_numpy(current).to(device), k, bs,
                           seed, truth)
    oracle = order == "oracle_current"
    _, _, _, got = t.run([gamma], order, True, oracle, 4)
    blocks = -(-length // bs)
    prev_max = np.full(blocks, -np.inf)
    prev_max[: t.prev_max.shape[1]] = t.prev_max.cpu().double().numpy()[0]
    upper = R.upper_bounds(prev_max, gamma, previous.size, length, bs)
    hot = np.zeros(blocks, dtype=bool)
    hot[np.minimum(t.seed_h // bs, blocks - 1)] = True
    cur_max = t.cur_max.cpu().double().numpy()[0]
    want = R.block_scan_order(order, cur_max if oracle else upper, cur_max, hot)
    np.testing.assert_array_equal(got[0], want)
    if gamma > 1e6 and not oracle:  # the case the packed sort cannot order alone
        kept_upper = upper[np.isfinite(upper)]
        assert np.unique(kept_upper.astype(np.float32)).size < np.unique(kept_upper).size
