"""Writes the verifier golden vectors from the reference package.

Run in the build container only (CPU, numpy):

    python tests/golden/make_verifier_vectors.py /root/reference/src

It imports ``temporal_dsa.verifier`` and ``temporal_dsa.approx`` from the
given source directory, runs ``verifier_step`` over small seeded
trajectories (temporal policies x verifier paths x promotion policies), and
writes ``verifier_vectors.npz`` (inputs, details and next-state arrays) and
``verifier_vectors.json`` (metrics dicts) next to this file.  The tests
compare the CPU restatement in ``oracle/verifier.py`` with these files;
nothing at test time imports the reference.

Why vectors: the reference's own verifier tests pin a handful of fields on
hand-built cases; the full metrics dict (byte accounting at three physical
block sizes, detector AP, retention at five depths, mass ratio) and the
rescued-state arrays over multi-step trajectories are pinned only here.
"""

from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

START = 300
STEPS = 6
K = 20
POLICIES = [
    dict(name="static", gamma=0.0),
    dict(name="dynamic_hot", gamma=0.1, dynamic_threshold=True, order="previous_max"),
    dict(name="ema", gamma=0.05, risk_model="ema", ema_alpha=0.8, volatility_lambda=0.5, age_slope=0.01),
]
CONFIGS = [
    dict(name="head8_b16", path="head", width=8, score_ratio=0.125, block_size=16, rescue_fraction=0.1),
    dict(name="head16_b32_keep", path="head", width=16, score_ratio=0.25, block_size=32, rescue_fraction=0.3,
         retain_candidate_keys=True),
    dict(name="dim16_b16", path="dim", width=16, score_ratio=0.125, block_size=16, rescue_fraction=0.05,
         sketch_bytes_per_token=8.0),
    dict(name="head8_none", path="head", width=8, score_ratio=0.125, block_size=16, rescue_fraction=0.0),
]
THRESHOLDS = [None, 1.0]


def make_trajectory(seed: int):
    """Dense score rows (growing by one key per step) and verifier rows that
    track them with noise, float32."""

    rng = np.random.default_rng(seed)
    length = START + STEPS
    current = rng.standard_normal(length).astype(np.float32)
    current[rng.choice(length, size=length // 30, replace=False)] += 2.5
    rows, partial = [], []
    for t in range(STEPS + 1):
        current = (0.9 * current + 0.45 * rng.standard_normal(length)).astype(np.float32)
        # a burst of newly active keys every other step
        if t % 2 == 1:
            burst = rng.integers(0, START - 32)
            current[burst : burst + 6] += 3.0
        rows.append(current[: START + t].copy())
        partial.append((0.6 * current[: START + t] + 0.3 * rng.standard_normal(START + t)).astype(np.float32))
    return rows, partial


def jsonable(value):
    if isinstance(value, np.integer):
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
    from temporal_dsa import verifier as ref_verifier

    arrays: dict[str, np.ndarray] = {}
    results: list[dict] = []
    case = 0
    for p_i, pspec in enumerate(POLICIES):
        policy = ref_approx.ApproxPolicy(**pspec)
        for c_i, cspec in enumerate(CONFIGS):
            config = ref_verifier.VerifierConfig(**cspec)
            for t_i, threshold in enumerate(THRESHOLDS):
                seed = 1582 + 100 * p_i + 10 * c_i + t_i
                rows, partial = make_trajectory(seed)
                for s, (r, v) in enumerate(zip(rows, partial)):
                    arrays[f"c{case}_scores_{s}"] = r
                    arrays[f"c{case}_verifier_{s}"] = v
                state = ref_approx.initialize_state(rows[0], k=K, block_size=config.block_size)
                steps = []
                for s in range(1, len(rows)):
                    tail = np.array([1, 5, 9], dtype=np.int64) if s == 2 else None
                    state, metrics, details = ref_verifier.verifier_step(
                        state, rows[s], partial[s], policy=policy, config=config, k=K, step=s,
                        previous_length=rows[s - 1].size, tail_critical_blocks=tail,
                        promotion_threshold=threshold,
                    )
                    for name in ("approximate", "rescued_blocks", "block_ranking", "exact_candidates"):
                        arrays[f"c{case}_{name}_{s}"] = np.asarray(details[name], dtype=np.int64)
                    for name in ("last_max", "ema", "volatility", "age", "cold_streak", "topk"):
                        arrays[f"c{case}_state_{name}_{s}"] = np.asarray(getattr(state, name))
                    steps.append({key: jsonable(val) for key, val in metrics.items()})
                results.append(dict(case=case, policy=pspec, config=cspec, threshold=threshold, seed=seed,
                                    k=K, steps=steps))
                case += 1
    np.savez_compressed(HERE / "verifier_vectors.npz", **arrays)
    (HERE / "verifier_vectors.json").write_text(json.dumps(results, indent=1, sort_keys=True) + "\n")
    print(f"wrote {case} cases")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
