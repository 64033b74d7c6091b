"""CPU restatement of the two-path verifier step (test oracle).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the HIP
verifier step, never by the product path.

Reference: verifier.py:15-432.  One decode step runs the own-trajectory
temporal filter (approx.replay_step, own history), then scans every key the
filter left unscored ("cold") with a cheap verifier score, ranks the blocks
holding cold keys by their largest cold verifier score (larger first, lower
block id on ties), rescues either the first ceil(rescue_fraction * cold
blocks) of that ranking or every ranked block at or above a fixed promotion
threshold, scores the rescued blocks in full, and takes the stable top-k of
the union of temporally scored keys and rescued blocks.  Only rescued blocks'
metadata sees the current scores (last max, EMA, volatility, age 0); the
cold streak of every block restarts from the final top-k.

``wave`` is passed through to the temporal filter (1 = the reference).

Pinned in tests/test_oracle_verifier.py: the reference's own hand cases
(rescue of a newly active block without duplicate scoring, no leakage from
an unrescued block, the cost identity, fixed-threshold promotion and its
address-stable ties) and golden vectors written from the reference
(tests/golden/make_verifier_vectors.py) over multi-step random trajectories
for both paths, both promotion policies and several temporal policies.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Callable

import numpy as np

from .approx import ApproxPolicy, ApproxState, initialize_state, replay_step
from .topk import stable_topk


@dataclass(frozen=True)
class VerifierConfig:
    """Reference: verifier.py:15-43 (same fields, defaults and checks)."""

    name: str
    path: str
    width: int
    score_ratio: float
    block_size: int = 64
    rescue_fraction: float = 0.05
    sketch_bytes_per_token: float = 0.0
    full_key_bytes_per_token: int = 256
    metadata_bytes_per_block: int = 4
    retain_candidate_keys: bool = False

    def __post_init__(self) -> None:
        if self.path not in {"head", "dim"}:
            raise ValueError("path must be 'head' or 'dim'")
        if self.width <= 0:
            raise ValueError("width must be positive")
        if not 0 <= self.rescue_fraction <= 1:
            raise ValueError("rescue_fraction must be in [0, 1]")
        if not 0 <= self.score_ratio <= 1:
            raise ValueError("score_ratio must be in [0, 1]")


def extend(values: np.ndarray, size: int, fill) -> np.ndarray:
    """First ``size`` entries of ``values``, padded with ``fill`` (verifier.py:46-49)."""

    values = np.asarray(values)
    out = np.full(size, fill, dtype=values.dtype)
    n = min(size, values.size)
    out[:n] = values[:n]
    return out


def block_max_masked(values: np.ndarray, available: np.ndarray, block_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Per block: the largest value among available keys (-inf if none) and
    whether any key is available (verifier.py:52-65)."""

    values = np.asarray(values, dtype=np.float32)
    n = values.size
    blocks = (n + block_size - 1) // block_size
    padded_v = np.full(blocks * block_size, -np.inf, dtype=np.float32)
    padded_v[:n] = values
    padded_a = np.zeros(blocks * block_size, dtype=bool)
    padded_a[:n] = np.asarray(available, dtype=bool)
    masked = np.where(padded_a, padded_v, -np.inf).reshape(blocks, block_size)
    return masked.max(axis=1).astype(np.float32), padded_a.reshape(blocks, block_size).any(axis=1)


def rank_blocks(scores: np.ndarray, eligible: np.ndarray) -> np.ndarray:
    """Eligible block ids by larger score, then lower id (verifier.py:68-73)."""

    ids = np.flatnonzero(eligible).astype(np.int64)
    if ids.size == 0:
        return ids
    return ids[np.lexsort((ids, -np.asarray(scores)[ids]))].astype(np.int64)


def average_precision(ranking: np.ndarray, positives: np.ndarray) -> float:
    """Average precision of a ranking against a positive set (verifier.py:76-86)."""

    wanted = set(int(v) for v in np.asarray(positives).ravel())
    if not wanted:
        return 1.0
    hit = np.isin(np.asarray(ranking, dtype=np.int64), np.fromiter(wanted, dtype=np.int64))
    ranks = np.flatnonzero(hit) + 1
    # sum over hits of (hits so far) / rank, in rank order
    total = 0.0
    for j, rank in enumerate(ranks.tolist(), start=1):
        total += j / rank
    return float(total / len(wanted))


def retention(approximate: np.ndarray, ranked_baseline: np.ndarray, count: int) -> float:
    """Share of the first ``count`` baseline keys that the selection holds (verifier.py:89-93)."""

    count = min(count, ranked_baseline.size)
    if count == 0:
        return 1.0
    return float(np.isin(ranked_baseline[:count], approximate).sum() / count)


def mass_ratio(scores: np.ndarray, approximate: np.ndarray, baseline: np.ndarray) -> float:
    """Softmax mass of the selection over the baseline's (verifier.py:96-100)."""

    shift = float(np.max(scores[baseline]))
    num = np.exp(scores[approximate].astype(np.float64) - shift).sum()
    den = np.exp(scores[baseline].astype(np.float64) - shift).sum()
    return float(num / max(den, 1e-300))


def _block_key_mask(blocks: np.ndarray, length: int, block_size: int) -> np.ndarray:
    mask = np.zeros(length, dtype=bool)
    for b in np.asarray(blocks, dtype=np.int64).tolist():
        mask[b * block_size : min(length, (b + 1) * block_size)] = True
    return mask


def apply_rescue_to_state(
    previous: ApproxState,
    temporal_next: ApproxState,
    scores,
    evaluated,
    rescued_blocks,
    *,
    policy: ApproxPolicy,
    k: int,
    block_size: int,
) -> tuple[ApproxState, np.ndarray, np.ndarray]:
    """Exact top-k of the candidate union and the rescued blocks' metadata
    (verifier.py:103-170)."""

    scores = np.asarray(scores, dtype=np.float32)
    length = scores.size
    rescued_blocks = np.asarray(rescued_blocks, dtype=np.int64)
    exact = _block_key_mask(rescued_blocks, length, block_size)
    exact[np.asarray(evaluated, dtype=np.int64)] = True
    exact_ids = np.flatnonzero(exact)
    if exact_ids.size < k:
        raise RuntimeError(f"candidate union has {exact_ids.size} keys, fewer than K={k}")
    approximate = exact_ids[stable_topk(scores[exact_ids], k)]

    nb = (length + block_size - 1) // block_size
    last_max = extend(temporal_next.last_max, nb, -math.inf).astype(np.float32)
    ema = extend(temporal_next.ema, nb, -math.inf).astype(np.float32)
    volatility = extend(temporal_next.volatility, nb, 0.0).astype(np.float32)
    age = extend(temporal_next.age, nb, 0).astype(np.int16)
    prev_ema = extend(previous.ema, nb, -math.inf).astype(np.float32)
    prev_vol = extend(previous.volatility, nb, 0.0).astype(np.float32)
    prev_cold = extend(previous.cold_streak, nb, 1).astype(np.int16)

    alpha = policy.ema_alpha
    for b in rescued_blocks.tolist():
        observed = float(np.max(scores[b * block_size : min(length, (b + 1) * block_size)]))
        mean = float(prev_ema[b]) if np.isfinite(prev_ema[b]) else observed
        last_max[b] = observed
        ema[b] = alpha * observed + (1.0 - alpha) * mean
        # numpy scalar rules: (1 - alpha) * float32 is float32, and the double
        # first term is added to it in float32.
        volatility[b] = alpha * abs(observed - mean) + (1.0 - alpha) * prev_vol[b]
        age[b] = 0

    hot = np.zeros(nb, dtype=bool)
    hot[approximate // block_size] = True
    cold = np.where(hot, 0, np.minimum(prev_cold.astype(np.int32) + 1, 32767)).astype(np.int16)
    state = ApproxState(
        topk=approximate,
        baseline_topk=temporal_next.baseline_topk,
        last_max=last_max,
        ema=ema,
        volatility=volatility,
        age=age,
        cold_streak=cold,
    )
    return state, approximate, exact_ids


def rescue_count(fraction: float, cold_blocks: int, ranked: int) -> int:
    """Blocks rescued under the global budget (verifier.py:208-212)."""

    return min(ranked, int(math.ceil(fraction * int(cold_blocks))))


def verifier_metrics(
    *,
    scores: np.ndarray,
    config: VerifierConfig,
    policy: ApproxPolicy,
    k: int,
    step: int,
    baseline: np.ndarray,
    temporal_evaluated: np.ndarray,
    cold_mask: np.ndarray,
    cold_blocks: np.ndarray,
    ranking: np.ndarray,
    rescued_blocks: np.ndarray,
    approximate: np.ndarray,
    exact_ids: np.ndarray,
    promotion_threshold: float | None,
    tail_critical_blocks=None,
) -> dict[str, Any]:
    """The metrics dict of one verifier step (verifier.py:227-391)."""

    length = scores.size
    bs = config.block_size
    base_mask = np.zeros(length, dtype=bool)
    base_mask[baseline] = True
    newly_active = baseline[cold_mask[baseline]]
    newly_active_blocks = np.unique(newly_active // bs)
    exact_mask = np.zeros(length, dtype=bool)
    exact_mask[exact_ids] = True
    rescued_token_hit = exact_mask[newly_active]
    rescued_positive = np.intersect1d(rescued_blocks, newly_active_blocks)
    tail = np.asarray([] if tail_critical_blocks is None else tail_critical_blocks, dtype=np.int64)
    rescued_tail = np.intersect1d(rescued_blocks, tail)

    temporal_exact = int(np.asarray(temporal_evaluated).size)
    rescue_new = int(exact_ids.size - temporal_exact)
    cold_tokens = int(cold_mask.sum())
    n_cold_blocks = int(np.asarray(cold_blocks).sum())
    full_equivalent = temporal_exact + rescue_new + cold_tokens * config.score_ratio
    nb = (length + bs - 1) // bs
    metadata_bytes = nb * config.metadata_bytes_per_block
    key_bytes = config.full_key_bytes_per_token
    temporal_key_bytes = temporal_exact * key_bytes
    if config.path == "head":
        verifier_key_bytes = cold_tokens * key_bytes
        reread = 0 if config.retain_candidate_keys else rescue_new * key_bytes
        sketch_bytes = 0.0
    else:
        verifier_key_bytes = 0.0
        sketch_bytes = cold_tokens * config.sketch_bytes_per_token
        reread = rescue_new * key_bytes
    total_key_bytes = temporal_key_bytes + verifier_key_bytes + sketch_bytes + reread + metadata_bytes
    baseline_key_bytes = length * key_bytes

    physical: dict[int, float] = {}
    for pb in (32, 64, 128):
        full_blocks = (length + pb - 1) // pb
        base_phys = full_blocks * pb * key_bytes
        if config.path == "head":
            reread_blocks = 0
            if not config.retain_candidate_keys and rescued_blocks.size:
                keys = np.flatnonzero(_block_key_mask(rescued_blocks, length, bs))
                reread_blocks = np.unique(keys // pb).size
            phys = base_phys + reread_blocks * pb * key_bytes + metadata_bytes
        else:
            exact_blocks = np.unique(np.flatnonzero(exact_mask) // pb).size
            cold_phys = np.unique(np.flatnonzero(cold_mask) // pb).size
            phys = exact_blocks * pb * key_bytes + cold_phys * pb * config.sketch_bytes_per_token + metadata_bytes
        physical[pb] = float(1.0 - phys / base_phys)

    return {
        "step": step,
        "context_length": length,
        "policy": policy.name,
        "verifier": config.name,
        "path": config.path,
        "width": config.width,
        "block_size": bs,
        "rescue_fraction": config.rescue_fraction,
        "promotion_policy": "global_budget" if promotion_threshold is None else "fixed_threshold",
        "promotion_threshold": math.nan if promotion_threshold is None else float(promotion_threshold),
        "promotion_fraction_of_cold": float(rescued_blocks.size / max(1, n_cold_blocks)),
        "temporal_exact_tokens": temporal_exact,
        "cold_tokens_scanned": cold_tokens,
        "cold_blocks_scanned": n_cold_blocks,
        "rescue_blocks": int(rescued_blocks.size),
        "rescue_exact_tokens": rescue_new,
        "candidate_union_tokens": int(exact_ids.size),
        "duplicate_exact_tokens": 0,
        "qk_full_equivalent": float(full_equivalent),
        "net_qk_reduction": float(1.0 - full_equivalent / float(length)),
        "exact_match": bool(np.array_equal(np.sort(approximate), np.sort(baseline))),
        "recall": float(base_mask[approximate].sum() / k),
        "top128_recall": retention(approximate, baseline, 128),
        "top256_recall": retention(approximate, baseline, 256),
        "top512_recall": retention(approximate, baseline, 512),
        "top1024_recall": retention(approximate, baseline, 1024),
        "top2048_recall": retention(approximate, baseline, 2048),
        "index_mass_ratio": mass_ratio(scores, approximate, baseline),
        "newly_active_tokens": int(newly_active.size),
        "newly_active_token_recall": float(rescued_token_hit.mean()) if newly_active.size else 1.0,
        "newly_active_blocks": int(newly_active_blocks.size),
        "newly_active_block_recall": (
            float(rescued_positive.size / newly_active_blocks.size) if newly_active_blocks.size else 1.0
        ),
        "detector_ap": average_precision(ranking, newly_active_blocks),
        "rescue_precision": float(rescued_positive.size / rescued_blocks.size) if rescued_blocks.size else 1.0,
        "tail_critical_blocks": int(tail.size),
        "tail_critical_block_recall": float(rescued_tail.size / tail.size) if tail.size else 1.0,
        "temporal_key_bytes": float(temporal_key_bytes),
        "verifier_key_bytes": float(verifier_key_bytes),
        "sketch_bytes": float(sketch_bytes),
        "rescue_reread_key_bytes": float(reread),
        "metadata_bytes": int(metadata_bytes),
        "total_key_bytes": float(total_key_bytes),
        "ideal_key_byte_reduction": float(1.0 - total_key_bytes / baseline_key_bytes),
        "physical_key_byte_reduction": physical[64],
        "physical_b32_key_byte_reduction": physical[32],
        "physical_b64_key_byte_reduction": physical[64],
        "physical_b128_key_byte_reduction": physical[128],
    }


def verifier_step(
    state: ApproxState,
    current_scores,
    verifier_scores,
    *,
    policy: ApproxPolicy,
    config: VerifierConfig,
    k: int,
    step: int,
    previous_length: int | None = None,
    tail_critical_blocks=None,
    promotion_threshold: float | None = None,
    wave: int = 1,
) -> tuple[ApproxState, dict[str, Any], dict[str, np.ndarray]]:
    """Temporal filter, current-query verification and exact rerank
    (verifier.py:173-392)."""

    scores = np.asarray(current_scores, dtype=np.float32)
    verifier_scores = np.asarray(verifier_scores, dtype=np.float32)[: scores.size]
    if verifier_scores.shape != scores.shape:
        raise ValueError("verifier score length must match current score length")
    temporal_next, _, detail = replay_step(
        state, scores, policy=policy, k=k, block_size=config.block_size, step=step,
        history_mode="own", previous_length=previous_length, wave=wave,
    )
    cold_mask = np.ones(scores.size, dtype=bool)
    cold_mask[detail["evaluated"]] = False
    block_scores, cold_blocks = block_max_masked(verifier_scores, cold_mask, config.block_size)
    ranking = rank_blocks(block_scores, cold_blocks)
    if promotion_threshold is None:
        rescued = ranking[: rescue_count(config.rescue_fraction, int(cold_blocks.sum()), ranking.size)]
    else:
        rescued = ranking[block_scores[ranking] >= float(promotion_threshold)]
    new_state, approximate, exact_ids = apply_rescue_to_state(
        state, temporal_next, scores, detail["evaluated"], rescued,
        policy=policy, k=k, block_size=config.block_size,
    )
    baseline = detail["baseline"]
    metrics = verifier_metrics(
        scores=scores, config=config, policy=policy, k=k, step=step, baseline=baseline,
        temporal_evaluated=detail["evaluated"], cold_mask=cold_mask, cold_blocks=cold_blocks,
        ranking=ranking, rescued_blocks=rescued, approximate=approximate, exact_ids=exact_ids,
        promotion_threshold=promotion_threshold, tail_critical_blocks=tail_critical_blocks,
    )
    newly_active = baseline[cold_mask[baseline]]
    details = {
        "approximate": approximate,
        "baseline": baseline,
        "temporal_approximate": detail["approximate"],
        "temporal_evaluated": detail["evaluated"],
        "cold": np.flatnonzero(cold_mask),
        "block_ranking": ranking,
        "block_scores": block_scores,
        "rescued_blocks": rescued,
        "exact_candidates": exact_ids,
        "newly_active": newly_active,
        "newly_active_blocks": np.unique(newly_active // config.block_size),
    }
    return new_state, metrics, details


def replay_verifier_trace(
    scores: np.ndarray,
    lengths: np.ndarray,
    verifier_scores: np.ndarray | Callable[[int, int], np.ndarray],
    *,
    policy: ApproxPolicy,
    config: VerifierConfig,
    k: int = 2048,
    max_transitions: int | None = None,
    tail_labels: dict[int, np.ndarray] | None = None,
    promotion_threshold: float | Callable[[int, int], float] | None = None,
    trace_info: dict[str, Any] | None = None,
) -> list[dict[str, Any]]:
    """One trace, step by step, with the verifier (verifier.py:395-432).
    ``scores`` [steps, Lmax] and ``lengths`` [steps] are the trace's rows."""

    lengths = np.asarray(lengths, dtype=np.int64)
    state = initialize_state(np.asarray(scores[0, : lengths[0]], dtype=np.float32), k=k, block_size=config.block_size)
    stop = scores.shape[0] if max_transitions is None else min(scores.shape[0], max_transitions + 1)
    rows: list[dict[str, Any]] = []
    info = dict(trace_info or {})
    for step in range(1, stop):
        length = int(lengths[step])
        partial = verifier_scores(step, length) if callable(verifier_scores) else verifier_scores[step, :length]
        thr = promotion_threshold(step, length) if callable(promotion_threshold) else promotion_threshold
        state, metrics, _ = verifier_step(
            state, np.asarray(scores[step, :length], dtype=np.float32), partial, policy=policy, config=config,
            k=k, step=step, previous_length=int(lengths[step - 1]),
            tail_critical_blocks=None if tail_labels is None else tail_labels.get(step),
            promotion_threshold=thr,
        )
        metrics.update(info)
        metrics["base_context_length"] = int(lengths[0]) - 1
        rows.append(metrics)
    return rows
