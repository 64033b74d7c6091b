"""Pins the own-trajectory oracle (oracle/approx.py) and the certified bound
(oracle/certified.py) with the reference's tests (reference
tests/test_approx.py:6-91, tests/test_certified.py:6-23) plus closed forms."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import scores as S
from oracle.approx import ApproxPolicy, initialize_state, replay_step
from oracle.certified import block_key_norms, temporal_score_radius
from oracle.topk import stable_topk


def test_full_refresh_matches_baseline_and_counts_every_key() -> None:
    previous = np.linspace(0, 1, 64, dtype=np.float32)
    current = previous[::-1].copy()
    state = initialize_state(previous, k=8, block_size=8)
    state, metrics, details = replay_step(state, current, policy=ApproxPolicy(name="full"), k=8, block_size=8, step=1, previous_length=64)
    assert metrics["exact_match"] and metrics["qk_scored"] == 64
    assert np.array_equal(np.sort(details["approximate"]), np.sort(details["baseline"]))


def test_seed_rescore_is_not_double_counted() -> None:
    previous = np.arange(64, dtype=np.float32)
    state = initialize_state(previous, k=8, block_size=8)
    _, metrics, _ = replay_step(state, previous.copy(), policy=ApproxPolicy(name="static", gamma=1e9), k=8, block_size=8, step=1, previous_length=64)
    assert metrics["qk_scored"] == 64


def test_own_trajectory_never_updates_skipped_block_with_truth() -> None:
    previous = np.zeros(32, dtype=np.float32)
    previous[:4] = 3
    state = initialize_state(previous, k=4, block_size=8)
    current = previous.copy()
    current[16:20] = 10
    state, metrics, _ = replay_step(state, current, policy=ApproxPolicy(name="static", gamma=0), k=4, block_size=8, step=1, previous_length=32)
    assert metrics["recall"] == 0
    assert state.last_max[2] == 0 and state.age[2] == 1


def test_age_cap_forces_stale_block_refresh() -> None:
    previous = np.zeros(32, dtype=np.float32)
    previous[:4] = 3
    state = initialize_state(previous, k=4, block_size=8)
    current = previous.copy()
    current[16:20] = 10
    policy = ApproxPolicy(name="age", gamma=0, age_cap=1)
    state, first, _ = replay_step(state, current, policy=policy, k=4, block_size=8, step=1, previous_length=32)
    state, second, _ = replay_step(state, current, policy=policy, k=4, block_size=8, step=2, previous_length=32)
    assert first["recall"] == 0 and second["recall"] == 1


def test_scattered_seed_physical_traffic_is_reported() -> None:
    previous = np.zeros(64, dtype=np.float32)
    previous[::8] = 5
    state = initialize_state(previous, k=8, block_size=8)
    _, metrics, _ = replay_step(state, previous.copy(), policy=ApproxPolicy(name="static", gamma=0), k=8, block_size=8, step=1, previous_length=64)
    assert metrics["seed_blocks_touched"] == 8 and metrics["physical_b16_blocks"] == 4


def test_dynamic_heap_returns_exact_topk_when_everything_is_scored() -> None:
    rng = np.random.default_rng(2)
    previous = rng.normal(size=200).astype(np.float32)
    current = np.round(rng.normal(size=200) * 3).astype(np.float32)  # ties
    state = initialize_state(previous, k=16, block_size=16)
    _, metrics, details = replay_step(state, current, policy=ApproxPolicy(name="d", dynamic_threshold=True, gamma=1e9), k=16, block_size=16, step=1)
    # gamma huge: nothing is skipped, the heap sees every key and must equal stable_topk
    assert metrics["exact_match"]
    assert np.array_equal(details["approximate"], stable_topk(current, 16))


def test_state_extends_for_new_blocks_and_cold_streak() -> None:
    previous = np.arange(16, dtype=np.float32)
    state = initialize_state(previous, k=2, block_size=4)
    assert state.cold_streak.tolist() == [1, 1, 1, 0]
    current = np.concatenate([previous, [100.0]])
    state2, metrics, details = replay_step(state, current, policy=ApproxPolicy(name="static", gamma=0), k=2, block_size=4, step=1, previous_length=16)
    assert state2.last_max.size == 5  # block 4 (the new key) was added and refreshed
    assert state2.last_max[4] == 100.0 and state2.age[4] == 0
    assert 4 in details["refreshed_blocks"].tolist()
    assert metrics["recall"] == 1.0


def test_rejects_short_seed() -> None:
    state = initialize_state(np.arange(8, dtype=np.float32), k=4, block_size=4)
    with pytest.raises(RuntimeError):
        replay_step(state, np.arange(6, dtype=np.float32), policy=ApproxPolicy(name="full"), k=4, block_size=4, step=1)


def test_temporal_radius_covers_every_key_with_signed_weights() -> None:
    rng = np.random.default_rng(1582)
    keys = rng.normal(size=(37, 8, 16))
    q_prev = rng.normal(size=(8, 16))
    q_now = q_prev + 0.05 * rng.normal(size=(8, 16))
    w_prev = rng.normal(size=8)
    w_now = w_prev + 0.05 * rng.normal(size=8)
    shared = keys[:, 0]
    before = S.relu_index_score(q_prev, shared, w_prev)
    after = S.relu_index_score(q_now, shared, w_now)
    norms = block_key_norms(np.repeat(shared[:, None, :], 8, axis=1), 7)
    radius = temporal_score_radius(q_now, q_prev, w_now, w_prev, norms)
    for block, start in enumerate(range(0, 37, 7)):
        assert np.all(np.abs(after[start : start + 7] - before[start : start + 7]) <= radius[block] + 1e-10)


def test_radius_closed_forms() -> None:
    rng = np.random.default_rng(5)
    q = rng.normal(size=(4, 8))
    w = rng.normal(size=4)
    norms = np.abs(rng.normal(size=(3, 4)))
    np.testing.assert_allclose(temporal_score_radius(q, q, w, w, norms), 0.0)
    # one head, weight change only: |dw| * ||q|| * n
    q1 = np.array([[3.0, 4.0]])
    r = temporal_score_radius(q1, q1, np.array([2.0]), np.array([-1.0]), np.array([[2.0]]))
    assert r.tolist() == [3.0 * 5.0 * 2.0]
    # one head, query change only: |w| * ||dq|| * n
    r = temporal_score_radius(np.array([[1.0, 1.0]]), np.array([[1.0, -2.0]]), np.array([-0.5]), np.array([-0.5]), np.array([[4.0]]))
    assert r.tolist() == [0.5 * 3.0 * 4.0]


def test_radius_asymmetric_closed_form() -> None:
    # Query and weight both change, ||q_now|| = 10 != ||q_prev|| = 5 and
    # |w_now| = 2 != |w_prev| = 1.  certified.py:43-47 fixes the form
    # |w_now - w_prev| ||q_prev|| + |w_now| ||q_now - q_prev|| = 3*5 + 2*5 = 25.
    # The plausible slips give other values: ||q_now|| in the first term 40,
    # |w_prev| in the second 20, both 35.
    q_now, q_prev = np.array([[6.0, 8.0]]), np.array([[3.0, 4.0]])
    w_now, w_prev = np.array([2.0]), np.array([-1.0])
    r = temporal_score_radius(q_now, q_prev, w_now, w_prev, np.array([[2.0], [0.5]]))
    assert r.tolist() == [50.0, 12.5]
    # Two heads with different block norms: the per-head coefficients are
    # weighted by their own head's norm (norms @ coefficients, not transposed).
    q_now2 = np.array([[6.0, 8.0], [0.0, 1.0]])
    q_prev2 = np.array([[3.0, 4.0], [0.0, 1.0]])
    r2 = temporal_score_radius(q_now2, q_prev2, np.array([2.0, 4.0]), np.array([-1.0, 1.0]), np.array([[2.0, 10.0]]))
    # head 0: 25 * 2; head 1: |4 - 1| * 1 + 4 * 0 = 3, * 10
    assert r2.tolist() == [50.0 + 30.0]


def test_block_key_norms_closed_form() -> None:
    keys = np.zeros((5, 2, 2))
    keys[0, 0] = [3, 4]  # norm 5
    keys[3, 0] = [6, 8]  # norm 10
    keys[1, 1] = [1, 0]
    out = block_key_norms(keys, 2)
    assert out.tolist() == [[5.0, 1.0], [10.0, 0.0], [0.0, 0.0]]


def test_approx_wave_covering_every_block_is_the_static_policy() -> None:
    # A threshold refreshed only after the whole scan never prunes anything
    # the seed threshold would not: the dynamic policy with one wave over all
    # blocks makes the static policy's decisions in the same order.
    rng = np.random.default_rng(9)
    previous = rng.normal(size=600).astype(np.float32)
    current = (0.9 * np.pad(previous, (0, 3)) + 0.3 * rng.normal(size=603)).astype(np.float32)
    for order, gamma in (("address", -0.4), ("previous_max", -0.2), ("bucket4", -0.6)):
        static = ApproxPolicy(name="s", gamma=gamma, order=order, cold_streak=0)
        dynamic = ApproxPolicy(name="d", gamma=gamma, order=order, cold_streak=0, dynamic_threshold=True)
        results = []
        for policy, wave in ((static, 1), (dynamic, 1000)):
            state = initialize_state(previous, k=32, block_size=16)
            state, metrics, details = replay_step(state, current, policy=policy, k=32, block_size=16, step=1,
                                                  previous_length=600, wave=wave)
            results.append((state, metrics, details))
        (s0, m0, d0), (s1, m1, d1) = results
        assert m0["blocks_skipped"] > 0, order
        np.testing.assert_array_equal(d0["refreshed_blocks"], d1["refreshed_blocks"])
        assert m0["qk_scored"] == m1["qk_scored"]
        assert sorted(d0["approximate"].tolist()) == sorted(d1["approximate"].tolist())
        for field in ("last_max", "ema", "volatility", "age", "cold_streak"):
            np.testing.assert_array_equal(getattr(s0, field), getattr(s1, field))
        # and a per-block refresh prunes at least as much as the seed threshold
        state = initialize_state(previous, k=32, block_size=16)
        _, m2, _ = replay_step(state, current, policy=dynamic, k=32, block_size=16, step=1, previous_length=600)
        assert m2["qk_scored"] <= m0["qk_scored"], order


def test_certified_margins_restate_the_radius_for_shared_keys() -> None:
    from oracle.certified import SCORE_ROUNDING_ALLOWANCE, certified_margins

    # One head, one key block: radius 3*5 + 2*5 = 25 per unit key norm (the
    # asymmetric closed form above), the block's largest key norm is 13
    # ((5, 12)), and the rounding allowance adds 2^-15 * 13 * (2*10 + 1*5).
    keys = np.array([[3.0, 4.0], [5.0, 12.0], [0.0, 1.0]])
    m = certified_margins(np.array([[6.0, 8.0]]), np.array([[3.0, 4.0]]), np.array([2.0]), np.array([-1.0]), keys, 4)
    assert m.tolist() == [25.0 * 13.0 + SCORE_ROUNDING_ALLOWANCE * 13.0 * 25.0]


def test_certified_margins_cover_every_key_change() -> None:
    from oracle.certified import certified_margins

    rng = np.random.default_rng(11)
    for rho in (0.9, 0.999):
        q_prev = rng.normal(size=(64, 128)) / np.sqrt(128)
        q_now = rho * q_prev + np.sqrt(1 - rho * rho) * rng.normal(size=(64, 128)) / np.sqrt(128)
        w_prev = rng.normal(size=64) / 8
        w_now = w_prev + 0.01 * rng.normal(size=64)
        keys = rng.normal(size=(500, 128))
        before = S.relu_index_score(q_prev, keys, w_prev)
        after = S.relu_index_score(q_now, keys, w_now)
        m = certified_margins(q_now, q_prev, w_now, w_prev, keys, 16)
        for b, start in enumerate(range(0, 500, 16)):
            assert np.all(np.abs(after[start : start + 16] - before[start : start + 16]) <= m[b])
