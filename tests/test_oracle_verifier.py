"""The CPU restatement of the two-path verifier step (oracle/verifier.py).

Pinned two ways:
  * the reference's own hand cases (reference tests/test_verifier.py:18-131):
    a newly active block is rescued without duplicate scoring and its
    metadata sees the current max; an unrescued block leaks nothing; the cost
    identity qk_full_equivalent = temporal + rescue + cold * ratio; a fixed
    threshold promotes exactly the blocks at or above it, ties stable by
    address;
  * golden vectors the reference wrote (tests/golden/make_verifier_vectors.py):
    24 multi-step trajectories over 3 temporal policies x 4 verifier configs
    (head/dim path, retained keys, zero budget) x 2 promotion policies.  Every
    metric, every detail array and every next-state array must match.
"""

from __future__ import annotations

import importlib.util
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import approx as A
from oracle import verifier as V

GOLDEN = Path(__file__).resolve().parent / "golden"
_spec = importlib.util.spec_from_file_location("make_verifier_vectors", GOLDEN / "make_verifier_vectors.py")
gen = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(gen)

RESULTS = json.loads((GOLDEN / "verifier_vectors.json").read_text())
ARRAYS = np.load(GOLDEN / "verifier_vectors.npz")


def _config(rescue_fraction: float = 0.5) -> V.VerifierConfig:
    return V.VerifierConfig(name="head8", path="head", width=8, score_ratio=0.125, block_size=8,
                            rescue_fraction=rescue_fraction)


def _newly_active_case():
    previous = np.zeros(32, dtype=np.float32)
    previous[:4] = 3
    current = previous.copy()
    current[16:20] = 10
    return previous, current


def test_rescues_newly_active_block_without_duplicate_scoring() -> None:
    previous, current = _newly_active_case()
    partial = np.zeros_like(current)
    partial[16:20] = 5
    state = A.initialize_state(previous, k=4, block_size=8)
    state, metrics, details = V.verifier_step(
        state, current, partial, policy=A.ApproxPolicy(name="static", gamma=0), config=_config(), k=4, step=1,
        previous_length=32,
    )
    assert metrics["recall"] == 1
    assert metrics["newly_active_token_recall"] == 1
    assert metrics["duplicate_exact_tokens"] == 0
    assert 2 in details["rescued_blocks"]
    assert state.last_max[2] == 10
    assert state.age[2] == 0


def test_unrescued_block_does_not_leak_current_score() -> None:
    previous, current = _newly_active_case()
    state = A.initialize_state(previous, k=4, block_size=8)
    state, metrics, _ = V.verifier_step(
        state, current, np.zeros_like(current), policy=A.ApproxPolicy(name="static", gamma=0),
        config=_config(rescue_fraction=0), k=4, step=1, previous_length=32,
    )
    assert metrics["recall"] == 0
    assert state.last_max[2] == 0
    assert state.age[2] == 1


def test_cost_includes_verifier_and_candidate_rerank() -> None:
    previous = np.arange(32, dtype=np.float32)
    state = A.initialize_state(previous, k=4, block_size=8)
    _, metrics, _ = V.verifier_step(
        state, previous.copy(), previous.copy(), policy=A.ApproxPolicy(name="static", gamma=1e9),
        config=_config(rescue_fraction=0.5), k=4, step=1, previous_length=32,
    )
    expected = metrics["temporal_exact_tokens"] + metrics["rescue_exact_tokens"] + metrics["cold_tokens_scanned"] * 0.125
    assert metrics["qk_full_equivalent"] == expected
    assert metrics["candidate_union_tokens"] == metrics["temporal_exact_tokens"] + metrics["rescue_exact_tokens"]
    assert metrics["physical_b64_key_byte_reduction"] <= 0


def test_fixed_threshold_promotes_all_blocks_at_or_above_cutoff() -> None:
    previous, current = _newly_active_case()
    verifier = np.zeros_like(current)
    verifier[8:16] = 4
    verifier[16:24] = 5
    state = A.initialize_state(previous, k=4, block_size=8)
    _, metrics, details = V.verifier_step(
        state, current, verifier, policy=A.ApproxPolicy(name="static", gamma=0), config=_config(rescue_fraction=0),
        k=4, step=1, previous_length=32, promotion_threshold=5,
    )
    assert metrics["promotion_policy"] == "fixed_threshold"
    assert metrics["promotion_threshold"] == 5
    np.testing.assert_array_equal(details["rescued_blocks"], [2])


def test_fixed_threshold_tie_break_is_block_address_stable() -> None:
    values = np.zeros(32, dtype=np.float32)
    values[:4] = 3
    state = A.initialize_state(values, k=4, block_size=8)
    _, _, details = V.verifier_step(
        state, values, np.ones_like(values), policy=A.ApproxPolicy(name="static", gamma=0),
        config=_config(rescue_fraction=0), k=4, step=1, previous_length=32, promotion_threshold=1,
    )
    np.testing.assert_array_equal(details["rescued_blocks"], np.arange(1, 4))


def test_config_validation() -> None:
    with pytest.raises(ValueError):
        V.VerifierConfig(name="x", path="rows", width=8, score_ratio=0.1)
    with pytest.raises(ValueError):
        V.VerifierConfig(name="x", path="head", width=0, score_ratio=0.1)
    with pytest.raises(ValueError):
        V.VerifierConfig(name="x", path="head", width=8, score_ratio=0.1, rescue_fraction=1.5)
    with pytest.raises(ValueError):
        V.VerifierConfig(name="x", path="head", width=8, score_ratio=2.0)


def test_rank_and_average_precision_closed_forms() -> None:
    scores = np.array([1.0, 3.0, 3.0, -np.inf, 2.0], dtype=np.float32)
    eligible = np.array([True, True, True, False, True])
    np.testing.assert_array_equal(V.rank_blocks(scores, eligible), [1, 2, 4, 0])
    # positives at ranks 1 and 3: (1/1 + 2/3) / 2
    assert V.average_precision(np.array([1, 2, 4, 0]), np.array([1, 4])) == pytest.approx((1 + 2 / 3) / 2, rel=1e-15)
    assert V.average_precision(np.array([1, 2]), np.array([], dtype=np.int64)) == 1.0
    assert V.rescue_count(0.1, 31, 31) == 4 and V.rescue_count(0.0, 31, 31) == 0 and V.rescue_count(1.0, 5, 3) == 3


def _same(expected, got) -> bool:
    if isinstance(expected, str) and expected in ("nan", "inf", "-inf"):
        return math.isnan(got) if expected == "nan" else got == float(expected)
    if isinstance(expected, bool) or isinstance(got, (bool, np.bool_)):
        return bool(expected) == bool(got)
    if isinstance(expected, int):
        return int(got) == expected
    if isinstance(expected, float):
        g = float(got)
        return g == expected or abs(g - expected) <= 1e-12 * max(1.0, abs(expected))
    return expected == got


@pytest.mark.parametrize("case", range(len(RESULTS)))
def test_verifier_step_matches_reference_vectors(case) -> None:
    spec = RESULTS[case]
    rows, partial = gen.make_trajectory(spec["seed"])
    if case == 0:
        for s, (r, v) in enumerate(zip(rows, partial)):
            np.testing.assert_array_equal(ARRAYS[f"c0_scores_{s}"], r)
            np.testing.assert_array_equal(ARRAYS[f"c0_verifier_{s}"], v)
    policy = A.ApproxPolicy(**spec["policy"])
    config = V.VerifierConfig(**spec["config"])
    k = spec["k"]
    state = A.initialize_state(rows[0], k=k, block_size=config.block_size)
    for s in range(1, len(rows)):
        tail = np.array([1, 5, 9], dtype=np.int64) if s == 2 else None
        state, metrics, details = V.verifier_step(
            state, rows[s], partial[s], policy=policy, config=config, k=k, step=s,
            previous_length=rows[s - 1].size, tail_critical_blocks=tail, promotion_threshold=spec["threshold"],
        )
        want = spec["steps"][s - 1]
        assert set(metrics) == set(want)
        for field, expected in want.items():
            assert _same(expected, metrics[field]), (case, s, field, expected, metrics[field])
        for name in ("approximate", "rescued_blocks", "block_ranking", "exact_candidates"):
            np.testing.assert_array_equal(details[name], ARRAYS[f"c{case}_{name}_{s}"], err_msg=f"{case} {s} {name}")
        for name in ("last_max", "ema", "volatility", "age", "cold_streak", "topk"):
            np.testing.assert_array_equal(getattr(state, name), ARRAYS[f"c{case}_state_{name}_{s}"],
                                          err_msg=f"{case} {s} {name}")


def test_replay_verifier_trace_rows_match_step_loop() -> None:
    rows, partial = gen.make_trajectory(77)
    width = max(r.size for r in rows)
    scores = np.full((len(rows), width), -np.inf, dtype=np.float32)
    verifier = np.zeros_like(scores)
    for s, (r, v) in enumerate(zip(rows, partial)):
        scores[s, : r.size] = r
        verifier[s, : v.size] = v
    lengths = np.array([r.size for r in rows])
    policy = A.ApproxPolicy(name="static", gamma=0.1)
    config = V.VerifierConfig(name="h", path="head", width=8, score_ratio=0.125, block_size=16, rescue_fraction=0.2)
    got = V.replay_verifier_trace(scores, lengths, verifier, policy=policy, config=config, k=16,
                                  trace_info={"layer": 3, "workload": "w", "prompt_id": "p"})
    state = A.initialize_state(rows[0], k=16, block_size=16)
    for s in range(1, len(rows)):
        state, metrics, _ = V.verifier_step(state, rows[s], partial[s], policy=policy, config=config, k=16, step=s,
                                            previous_length=rows[s - 1].size)
        assert {key: got[s - 1][key] for key in metrics} == metrics
        assert got[s - 1]["layer"] == 3 and got[s - 1]["base_context_length"] == rows[0].size - 1
