"""The CPU restatement of replay / approx against vectors the reference wrote.

``tests/golden/replay_vectors.{json,npz}`` hold ReplayResult rows of
``replay_transition`` (reference replay.py:225-400), the per-transition and
aggregated tables of ``replay_trace`` (replay.py:476-627), and the metrics and
detail arrays of ``approx.replay_step`` (approx.py:129-364) on seeded synthetic
traces, written by ``tests/golden/make_replay_vectors.py`` from the reference
package in the build container.  Integer fields and index arrays must match
exactly; float fields to 1e-12 relative (same float64 / float32 arithmetic).
"""

from __future__ import annotations

import dataclasses
import importlib.util
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import approx as A
from oracle import replay as R

GOLDEN = Path(__file__).resolve().parent / "golden"
_spec = importlib.util.spec_from_file_location("make_replay_vectors", GOLDEN / "make_replay_vectors.py")
gen = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(gen)

RESULTS = json.loads((GOLDEN / "replay_vectors.json").read_text())
ARRAYS = np.load(GOLDEN / "replay_vectors.npz")


def same(expected, got) -> bool:
    if isinstance(expected, str) and expected in ("nan", "inf", "-inf"):
        return (math.isnan(got) if expected == "nan" else got == float(expected))
    if isinstance(expected, bool) or isinstance(got, (bool, np.bool_)):
        return bool(expected) == bool(got)
    if isinstance(expected, int) and not isinstance(expected, bool):
        return int(got) == expected
    if isinstance(expected, float):
        g = float(got)
        return g == expected or abs(g - expected) <= 1e-12 * max(1.0, abs(expected))
    return expected == got


@pytest.mark.parametrize("t", range(len(gen.TRANSITIONS)))
def test_replay_transition_matches_reference_vectors(t) -> None:
    previous = ARRAYS[f"replay_prev_{t}"]
    current = ARRAYS[f"replay_cur_{t}"]
    regen_previous, regen_current = gen.make_transition(1582 + t, *gen.TRANSITIONS[t])
    np.testing.assert_array_equal(previous, regen_previous)
    np.testing.assert_array_equal(current, regen_current)
    rows = [r for r in RESULTS["replay"] if r["transition"] == t]
    assert rows
    for row in rows:
        got = R.replay_transition(
            previous, current, k=row["k"], block_size=row["block_size"], gamma_sigma=row["gamma_sigma"],
            method=row["method"], scan_order=row["requested_order"], step=row["step"],
        )
        got = dataclasses.asdict(got)
        for field, expected in row.items():
            if field in ("transition", "requested_order"):
                continue
            assert same(expected, got[field]), (row["method"], row["requested_order"], row["k"], row["block_size"], row["gamma_sigma"], field, expected, got[field])


@pytest.mark.parametrize("p", range(len(gen.APPROX_POLICIES)))
@pytest.mark.parametrize("history", ["own", "teacher"])
def test_approx_replay_step_matches_reference_vectors(p, history) -> None:
    steps = gen.make_trace(2000 + p)
    if p == 0:
        for i, s in enumerate(steps):
            np.testing.assert_array_equal(ARRAYS[f"approx_trace_{i}"], s)
    policy = A.ApproxPolicy(**gen.APPROX_POLICIES[p])
    rows = [r for r in RESULTS["approx"] if r["policy_index"] == p and r["history_mode"] == history]
    assert len(rows) == len(steps) - 1
    state = A.initialize_state(steps[0], k=gen.APPROX_K, block_size=gen.APPROX_BLOCK)
    for i in range(1, len(steps)):
        state, metrics, details = A.replay_step(
            state, steps[i], policy=policy, k=gen.APPROX_K, block_size=gen.APPROX_BLOCK, step=i,
            history_mode=history, previous_length=steps[i - 1].size,
        )
        row = rows[i - 1]
        assert row["step"] == i
        for field, expected in row.items():
            if field == "policy_index":
                continue
            assert field in metrics, field
            assert same(expected, metrics[field]), (p, history, i, field, expected, metrics[field])
        assert set(metrics) == set(row) - {"policy_index"}
        for name in ("approximate", "evaluated", "refreshed_blocks", "skipped_blocks", "missed_ranks"):
            np.testing.assert_array_equal(np.asarray(details[name]), ARRAYS[f"approx_{p}_{history}_{i}_{name}"], err_msg=f"{p} {history} {i} {name}")
    for name in ("topk", "last_max", "age", "cold_streak"):
        np.testing.assert_array_equal(np.asarray(getattr(state, name)), ARRAYS[f"approx_{p}_{history}_state_{name}"], err_msg=name)


def test_replay_trace_rows_and_summary_match_reference_vectors() -> None:
    scores, lengths = gen.make_score_rows(4242)
    np.testing.assert_array_equal(ARRAYS["trace_scores"], scores)
    rows = [scores[t, : lengths[t]].astype(np.float32) for t in range(len(lengths))]
    kwargs = dict(k_values=gen.TRACE_K, block_sizes=gen.TRACE_BLOCKS, gamma_sigma_values=gen.TRACE_GAMMAS,
                  absolute_margins=gen.TRACE_MARGINS, layer=3, workload="synthetic", prompt_id="p7")
    got = R.replay_trace_rows(rows, **kwargs)
    want = RESULTS["trace_rows"]
    assert len(got) == len(want)
    for g, w in zip(got, want):
        assert set(g) == set(w)
        for field, expected in w.items():
            assert same(expected, g[field]), (w["step"], w["k"], w["block_size"], w["method"], w["scan_order"], field, expected, g[field])
    summary = R.aggregate_rows(got).to_dict("records")
    want_summary = RESULTS["trace_summary"]
    assert len(summary) == len(want_summary)
    for g, w in zip(summary, want_summary):
        assert set(g) == set(w)
        for field, expected in w.items():
            assert same(expected, g[field]), (w["k"], w["block_size"], w["method"], w["scan_order"], field, expected, g[field])
