"""GPU own-trajectory replay over recorded rows against the reference's output.

``tests/golden/replay_vectors.{json,npz}`` hold the reference's
``approx.replay_step`` (approx.py:129-364) metrics, details and final state
over 10-step float32 trajectories for 7 policies (written by the reference
itself, tests/golden/make_replay_vectors.py).  ``dsa_amd.approx.replay_step``
runs each transition in the HIP kernels with the recorded row as the score
source (``dsa_approx_replay_step``).  For both history modes ("own": seeds
and state follow the step's own top-k; "teacher": they follow the dense
trace), every metric, every detail array and the final state must match
exactly.
"""

from __future__ import annotations

import importlib.util
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from dsa_amd import approx

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
_spec = importlib.util.spec_from_file_location("make_replay_vectors", GOLDEN / "make_replay_vectors.py")
gen = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(gen)
RESULTS = json.loads((GOLDEN / "replay_vectors.json").read_text())
ARRAYS = np.load(GOLDEN / "replay_vectors.npz")


def same(expected, got) -> bool:
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


@pytest.mark.parametrize("history", ["own", "teacher"])
@pytest.mark.parametrize("p", range(len(gen.APPROX_POLICIES)))
def test_replay_step_matches_reference_vectors(device, p, history) -> None:
    spec = gen.APPROX_POLICIES[p]
    steps = gen.make_trace(2000 + p)
    policy = approx.ApproxPolicy(**spec)
    rows = [r for r in RESULTS["approx"] if r["policy_index"] == p and r["history_mode"] == history]
    assert len(rows) == len(steps) - 1
    state = approx.initialize_state(torch.from_numpy(steps[0]).to(device).reshape(1, -1), k=gen.APPROX_K,
                                    block_size=gen.APPROX_BLOCK, capacity=steps[-1].size)
    for i in range(1, len(steps)):
        state, metrics, details = approx.replay_step(
            state, steps[i], policy=policy, k=gen.APPROX_K, block_size=gen.APPROX_BLOCK, step=i,
            history_mode=history, previous_length=steps[i - 1].size)
        row = rows[i - 1]
        for field, expected in row.items():
            if field == "policy_index":
                continue
            assert same(expected, metrics[field]), (p, i, field, expected, metrics[field])
        assert set(metrics) == set(row) - {"policy_index"}
        for name in ("approximate", "evaluated", "refreshed_blocks", "skipped_blocks", "missed_ranks"):
            np.testing.assert_array_equal(np.asarray(details[name]), ARRAYS[f"approx_{p}_{history}_{i}_{name}"],
                                          err_msg=f"{p} {i} {name}")
    host = state.host()
    np.testing.assert_array_equal(state.seed_order, ARRAYS[f"approx_{p}_{history}_state_topk"])
    for name in ("last_max", "age", "cold_streak"):
        np.testing.assert_array_equal(host[name][0], ARRAYS[f"approx_{p}_{history}_state_{name}"], err_msg=name)
