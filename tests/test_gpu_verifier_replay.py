"""GPU verifier replay over recorded rows against the reference's own output.

``tests/golden/verifier_vectors.{json,npz}`` hold 24 multi-step trajectories
of the reference's ``verifier_step`` (3 temporal policies x 4 verifier
configs x 2 promotion policies), written by the reference itself
(tests/golden/make_verifier_vectors.py).  ``dsa_amd.verifier`` replays each on
the GPU (``dsa_verifier_replay_step``: the temporal scan, cold-block ranking,
rescue, union top-k and state update in the HIP kernels, with the recorded
rows as the score source).  Every metric of every step, the rescued blocks,
the ranking, the union and every next-state array must match exactly, and
``replay_verifier_trace`` must give the same rows as a DataFrame.
"""

from __future__ import annotations

import importlib.util
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from dsa_amd import approx, verifier
from dsa_amd.trace import ScoreTrace

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
_spec = importlib.util.spec_from_file_location("make_verifier_vectors", GOLDEN / "make_verifier_vectors.py")
gen = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(gen)
RESULTS = json.loads((GOLDEN / "verifier_vectors.json").read_text())
ARRAYS = np.load(GOLDEN / "verifier_vectors.npz")


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


def _case(case):
    spec = RESULTS[case]
    rows, partial = gen.make_trajectory(spec["seed"])
    policy = approx.ApproxPolicy(**spec["policy"])
    config = verifier.VerifierConfig(**spec["config"])
    return spec, rows, partial, policy, config


@pytest.mark.parametrize("case", range(len(RESULTS)))
def test_verifier_replay_step_matches_reference_vectors(device, case) -> None:
    spec, rows, partial, policy, config = _case(case)
    k = spec["k"]
    state = approx.initialize_state(torch.from_numpy(rows[0]).to(device).reshape(1, -1), k=k,
                                    block_size=config.block_size, capacity=rows[-1].size)
    for s in range(1, len(rows)):
        cur = torch.from_numpy(rows[s]).to(device).reshape(1, -1)
        ver = torch.from_numpy(partial[s]).to(device).reshape(1, -1)
        out = verifier.verifier_replay_step(state, cur, ver, policy=policy, config=config, step=s,
                                            promotion_threshold=spec["threshold"])
        tail = np.array([1, 5, 9], dtype=np.int64) if s == 2 else None
        metrics = verifier.verifier_metrics(out, cur, config=config, policy=policy, step=s,
                                            promotion_threshold=spec["threshold"], tail_critical_blocks=tail)
        want = spec["steps"][s - 1]
        assert set(metrics) == set(want)
        for field, expected in want.items():
            assert same(expected, metrics[field]), (case, s, field, expected, metrics[field])
        np.testing.assert_array_equal(np.sort(out.topk[0].cpu().numpy()), np.sort(ARRAYS[f"c{case}_approximate_{s}"]))
        np.testing.assert_array_equal(np.flatnonzero(out.rescued_blocks[0].cpu().numpy()),
                                      np.sort(ARRAYS[f"c{case}_rescued_blocks_{s}"]))
        ranking = out.ranking[0].cpu().numpy()
        np.testing.assert_array_equal(ranking[ranking >= 0], ARRAYS[f"c{case}_block_ranking_{s}"])
        np.testing.assert_array_equal(np.flatnonzero(np.isfinite(out.scores[0].cpu().numpy())),
                                      ARRAYS[f"c{case}_exact_candidates_{s}"])
        host = state.host()
        for name in ("last_max", "ema", "volatility", "age", "cold_streak"):
            np.testing.assert_array_equal(host[name][0], ARRAYS[f"c{case}_state_{name}_{s}"], err_msg=f"{case} {s} {name}")


@pytest.mark.parametrize("case", [0, 9, 17])
def test_replay_verifier_trace_frame_matches_reference(device, case) -> None:
    spec, rows, partial, policy, config = _case(case)
    width = rows[-1].size
    scores = np.full((len(rows), width), -np.inf, dtype=np.float32)
    ver = np.zeros((len(rows), width), dtype=np.float32)
    for s, (r, v) in enumerate(zip(rows, partial)):
        scores[s, : r.size] = r
        ver[s, : v.size] = v
    trace = ScoreTrace(scores=scores, lengths=np.array([r.size for r in rows]), layer=4, workload="w", prompt_id="p",
                       metadata={})
    frame = verifier.replay_verifier_trace(trace, ver, policy=policy, config=config, k=spec["k"],
                                           promotion_threshold=spec["threshold"],
                                           tail_labels={2: np.array([1, 5, 9], dtype=np.int64)})
    assert len(frame) == len(rows) - 1
    for s, row in enumerate(frame.to_dict("records"), start=1):
        for field, expected in spec["steps"][s - 1].items():
            assert same(expected, row[field]), (case, s, field, expected, row[field])
        assert row["layer"] == 4 and row["base_context_length"] == rows[0].size - 1
