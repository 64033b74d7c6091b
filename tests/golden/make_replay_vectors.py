"""Writes the replay / approx golden vectors from the reference package.

Run in the build container only (CPU, numpy):

    python tests/golden/make_replay_vectors.py /root/reference/src

It imports ``temporal_dsa.replay`` and ``temporal_dsa.approx`` from the given
source directory, runs them on small seeded synthetic traces, and writes
``replay_vectors.npz`` (inputs and output arrays) and ``replay_vectors.json``
(scalar results) next to this file.  The tests compare the CPU restatement in
``oracle/`` with these files; nothing at test time imports the reference.

Which results need vectors: ``replay_transition``'s ReplayResult fields,
``replay_trace``'s per-transition and aggregated tables, and
``approx.replay_step``'s metrics and detail arrays on random traces (reference
replay.py:225-400, replay.py:476-627, approx.py:129-364); hand cases pin only
a few of them.
"""

from __future__ import annotations

import dataclasses
import json
import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

# Transitions: (previous length, current length); previous ~ N(0,1) with hot
# keys, current = 0.9 * previous + 0.44 * noise on the shared prefix, fresh
# keys on the appended tail.
TRANSITIONS = [(500, 503), (640, 640), (777, 790)]
REPLAY_K = [16, 64]
REPLAY_BLOCKS = [16, 64]
REPLAY_GAMMAS = [0.0, 0.5]
REPLAY_METHODS = [
    ("full", "address"),
    ("static", "address"),
    ("static_hot_first", "previous_hot"),
    ("dynamic", "address"),
    ("dynamic", "previous_hot"),
    ("dynamic", "upper_hot"),
    ("oracle", "oracle_current"),
]

# Own-trajectory runs: 10 steps from length 400, one key appended per step.
APPROX_START = 400
APPROX_STEPS = 10
APPROX_K = 24
APPROX_BLOCK = 16
APPROX_POLICIES = [
    dict(name="full"),
    dict(name="static", gamma=0.0),
    dict(name="static_margin", gamma=0.4),
    dict(name="dynamic_hot", gamma=0.2, dynamic_threshold=True, order="previous_max"),
    dict(name="bucket", gamma=0.1, order="bucket4", cold_streak=2),
    dict(name="ema", gamma=0.1, risk_model="ema", ema_alpha=0.8, volatility_lambda=0.5, age_slope=0.01),
    dict(name="aged", gamma=0.0, age_cap=3, recent_window=20, refresh_interval=5),
    dict(name="oracle", gamma=0.0, dynamic_threshold=True, order="oracle_current"),
]


def make_transition(seed: int, previous_length: int, current_length: int):
    rng = np.random.default_rng(seed)
    previous = rng.standard_normal(previous_length)
    hot = rng.choice(previous_length, size=max(1, previous_length // 50), replace=False)
    previous[hot] += 3.0
    current = np.empty(current_length)
    current[:previous_length] = 0.9 * previous + 0.44 * rng.standard_normal(previous_length)
    current[previous_length:] = rng.standard_normal(current_length - previous_length)
    return previous, current


# replay_trace sweep: 5 steps from length 300, float32 rows like ScoreTrace.row.
TRACE_START = 300
TRACE_STEPS = 5
TRACE_K = [8, 32, 400]
TRACE_BLOCKS = [16, 32]
TRACE_GAMMAS = [0.0, 0.5]
TRACE_MARGINS = {16: 0.3}


def make_score_rows(seed: int):
    rng = np.random.default_rng(seed)
    width = TRACE_START + TRACE_STEPS - 1
    scores = np.full((TRACE_STEPS, width), -np.inf, dtype=np.float32)
    current = rng.standard_normal(width)
    current[rng.choice(width, size=width // 30, replace=False)] += 2.5
    for t in range(TRACE_STEPS):
        current = 0.93 * current + 0.37 * rng.standard_normal(width)
        scores[t, : TRACE_START + t] = current[: TRACE_START + t]
    lengths = np.arange(TRACE_START, TRACE_START + TRACE_STEPS)
    return scores, lengths


def make_trace(seed: int):
    rng = np.random.default_rng(seed)
    length = APPROX_START + APPROX_STEPS
    steps = []
    base = rng.standard_normal(length).astype(np.float32)
    base[rng.choice(length, size=length // 40, replace=False)] += 3.0
    current = base.copy()
    for t in range(APPROX_STEPS + 1):
        current = (0.92 * current + 0.39 * rng.standard_normal(length)).astype(np.float32)
        steps.append(current[: APPROX_START + t].copy())
    return steps


def jsonable(value):
    if isinstance(value, (np.integer,)):
        return int(value)
    if isinstance(value, (np.floating, float)):
        v = float(value)
        return "nan" if math.isnan(v) else ("inf" if v == math.inf else ("-inf" if v == -math.inf else v))
    if isinstance(value, (np.bool_, bool)):
        return bool(value)
    return value


def main(source: str) -> None:
    sys.path.insert(0, source)
    from temporal_dsa import approx as ref_approx
    from temporal_dsa import replay as ref_replay

    arrays: dict[str, np.ndarray] = {}
    results: dict[str, object] = {"replay": [], "approx": []}
    for t, (lp, lc) in enumerate(TRANSITIONS):
        previous, current = make_transition(1582 + t, lp, lc)
        arrays[f"replay_prev_{t}"] = previous
        arrays[f"replay_cur_{t}"] = current
        for k in REPLAY_K:
            for block in REPLAY_BLOCKS:
                for gamma in REPLAY_GAMMAS:
                    for method, order in REPLAY_METHODS:
                        r = ref_replay.replay_transition(
                            previous, current, k=k, block_size=block, gamma_sigma=gamma,
                            method=method, scan_order=order, step=t,
                        )
                        row = {key: jsonable(v) for key, v in dataclasses.asdict(r).items()}
                        row["transition"] = t
                        row["requested_order"] = order
                        results["replay"].append(row)

    from temporal_dsa.trace import ScoreTrace

    scores, lengths = make_score_rows(4242)
    arrays["trace_scores"] = scores
    arrays["trace_lengths"] = lengths
    trace = ScoreTrace(scores=scores, lengths=lengths, layer=3, workload="synthetic", prompt_id="p7", metadata={})
    kwargs = dict(k_values=TRACE_K, block_sizes=TRACE_BLOCKS, gamma_sigma_values=TRACE_GAMMAS,
                  absolute_margins=TRACE_MARGINS)
    per_step = ref_replay.replay_trace(trace, aggregate=False, **kwargs)
    summary = ref_replay.replay_trace(trace, aggregate=True, **kwargs)
    results["trace_rows"] = [{key: jsonable(v) for key, v in row.items()} for row in per_step.to_dict("records")]
    results["trace_summary"] = [{key: jsonable(v) for key, v in row.items()} for row in summary.to_dict("records")]

    for p, spec in enumerate(APPROX_POLICIES):
        for history in ("own", "teacher"):
            steps = make_trace(2000 + p)
            if p == 0 and history == "own":
                for i, s in enumerate(steps):
                    arrays[f"approx_trace_{i}"] = s
            policy = ref_approx.ApproxPolicy(**spec)
            state = ref_approx.initialize_state(steps[0], k=APPROX_K, block_size=APPROX_BLOCK)
            for i in range(1, len(steps)):
                state, metrics, details = ref_approx.replay_step(
                    state, steps[i], policy=policy, k=APPROX_K, block_size=APPROX_BLOCK, step=i,
                    history_mode=history, previous_length=steps[i - 1].size,
                )
                row = {key: jsonable(v) for key, v in metrics.items()}
                row["policy_index"] = p
                results["approx"].append(row)
                for name in ("approximate", "evaluated", "refreshed_blocks", "skipped_blocks", "missed_ranks"):
                    arrays[f"approx_{p}_{history}_{i}_{name}"] = np.asarray(details[name])
            for name in ("topk", "last_max", "age", "cold_streak"):
                arrays[f"approx_{p}_{history}_state_{name}"] = np.asarray(getattr(state, name))

    np.savez_compressed(HERE / "replay_vectors.npz", **arrays)
    (HERE / "replay_vectors.json").write_text(json.dumps(results, sort_keys=True, separators=(",", ":")) + "\n")
    print(f"wrote {len(results['replay'])} replay rows, {len(results['trace_rows'])} trace rows, "
          f"{len(results['trace_summary'])} summary rows, {len(results['approx'])} approx rows, {len(arrays)} arrays")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
