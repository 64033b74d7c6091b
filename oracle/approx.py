"""CPU restatement of the own-trajectory temporal policy (test oracle).

Reference: approx.py:15-364 (ApproxPolicy, ApproxState, initialize_state,
replay_step).  Per-block metadata (last max, EMA, volatility, age, cold
streak) is updated only for blocks that were refreshed, so skipped blocks keep
stale values and never see the current step's scores.

One extension, as in the replay oracle: ``wave``.  The reference refreshes the
running top-K threshold after every kept block; with ``wave = W`` the scan
order is cut into consecutive groups of W blocks, every block of a group is
skipped or refreshed against the threshold in force at the start of the
group, and the running top-K takes the group's new keys after it.  ``wave = 1``
is the reference schedule.
"""

from __future__ import annotations

import heapq
import math
from dataclasses import dataclass, replace
from typing import Any

import numpy as np

from .topk import stable_topk


@dataclass(frozen=True)
class ApproxPolicy:
    """Reference: approx.py:15-39 (same fields and defaults)."""

    name: str
    gamma: float = 0.0
    cold_streak: int = 1
    dynamic_threshold: bool = False
    order: str = "address"
    refresh_interval: int | None = None
    age_cap: int | None = None
    recent_window: int = 0
    risk_model: str = "last_max"
    ema_alpha: float = 0.9
    volatility_lambda: float = 0.0
    age_slope: float = 0.0
    fallback_threshold: float | None = None

    def with_gamma(self, gamma: float) -> "ApproxPolicy":
        return replace(self, gamma=float(gamma))


@dataclass
class ApproxState:
    """Reference: approx.py:42-50."""

    topk: np.ndarray
    baseline_topk: np.ndarray
    last_max: np.ndarray
    ema: np.ndarray
    volatility: np.ndarray
    age: np.ndarray
    cold_streak: np.ndarray


def block_max_f32(values: np.ndarray, block_size: int) -> np.ndarray:
    """Reference: approx.py:53-55."""

    values = np.asarray(values, dtype=np.float32)
    blocks = (values.size + block_size - 1) // block_size
    return np.array([values[b * block_size : (b + 1) * block_size].max() for b in range(blocks)], dtype=np.float32)


def _grow(values: np.ndarray, size: int, fill) -> np.ndarray:
    """Reference: approx.py:58-61."""

    out = np.full(size, fill, dtype=values.dtype)
    n = min(size, values.size)
    out[:n] = values[:n]
    return out


def metadata_bytes_per_block(policy: ApproxPolicy) -> int:
    """Reference: approx.py:84-90."""

    raw = 6 + (1 if policy.order.startswith("bucket") else 0) + (8 if policy.risk_model == "ema" else 0)
    return int(math.ceil(raw / 4) * 4)


def order_blocks(policy: ApproxPolicy, risk: np.ndarray) -> np.ndarray:
    """Reference: approx.py:93-109."""

    n = risk.size
    score = np.where(np.isnan(risk), -np.inf, risk)
    by_risk = sorted(range(n), key=lambda b: (-score[b], b))
    if policy.order == "address":
        return np.arange(n, dtype=np.int64)
    if policy.order in {"previous_max", "predicted_risk"}:
        return np.asarray(by_risk, dtype=np.int64)
    if policy.order.startswith("bucket"):
        buckets = int(policy.order[len("bucket"):])
        rank = np.empty(n, dtype=np.int64)
        rank[np.asarray(by_risk, dtype=np.int64)] = np.arange(n)
        bucket = np.minimum(buckets - 1, rank * buckets // max(1, n))
        return np.asarray(sorted(range(n), key=lambda b: (bucket[b], b)), dtype=np.int64)
    if policy.order == "oracle_current":
        raise ValueError("oracle order must be supplied with current block maxima")
    raise ValueError(f"unknown block order: {policy.order}")


def initialize_state(scores, *, k: int, block_size: int) -> ApproxState:
    """Reference: approx.py:112-126."""

    scores = np.asarray(scores, dtype=np.float32)
    top = stable_topk(scores, k)
    maxima = block_max_f32(scores, block_size)
    hot = np.zeros(maxima.size, dtype=bool)
    hot[top // block_size] = True
    return ApproxState(
        topk=top,
        baseline_topk=top.copy(),
        last_max=maxima,
        ema=maxima.copy(),
        volatility=np.zeros(maxima.size, dtype=np.float32),
        age=np.zeros(maxima.size, dtype=np.int16),
        cold_streak=np.where(hot, 0, 1).astype(np.int16),
    )


def _retention(approximate: np.ndarray, ranked: np.ndarray, count: int) -> float:
    count = min(count, ranked.size)
    return float(np.isin(ranked[:count], approximate).sum() / count)


def _mass_ratio(scores: np.ndarray, approximate: np.ndarray, baseline: np.ndarray) -> float:
    shift = float(np.max(scores[baseline]))
    num = np.exp(scores[approximate].astype(np.float64) - shift).sum()
    den = np.exp(scores[baseline].astype(np.float64) - shift).sum()
    return float(num / max(den, 1e-300))


def replay_step(
    state: ApproxState,
    current_scores,
    *,
    policy: ApproxPolicy,
    k: int,
    block_size: int,
    step: int,
    history_mode: str = "own",
    previous_length: int | None = None,
    fallback_value: float | None = None,
    wave: int = 1,
) -> tuple[ApproxState, dict[str, Any], dict[str, np.ndarray]]:
    """One own-trajectory transition.  Reference: approx.py:129-364."""

    if history_mode not in {"own", "teacher"}:
        raise ValueError("history_mode must be 'own' or 'teacher'")
    scores = np.asarray(current_scores, dtype=np.float32)
    length = scores.size
    if k > length:
        raise ValueError("K cannot exceed the current trace length")
    previous_length = length if previous_length is None else int(previous_length)
    blocks = (length + block_size - 1) // block_size
    last_max = _grow(np.asarray(state.last_max, dtype=np.float32), blocks, -np.inf)
    ema = _grow(np.asarray(state.ema, dtype=np.float32), blocks, -np.inf)
    volatility = _grow(np.asarray(state.volatility, dtype=np.float32), blocks, 0.0)
    age = _grow(np.asarray(state.age, dtype=np.int16), blocks, 0)
    cold = _grow(np.asarray(state.cold_streak, dtype=np.int16), blocks, 1)

    baseline = stable_topk(scores, k)
    seed = np.asarray(state.baseline_topk if history_mode == "teacher" else state.topk)
    seed = seed[seed < length].astype(np.int64)
    if seed.size != k or np.unique(seed).size != k:
        raise RuntimeError(f"previous Top-K seed has {seed.size} unique keys, expected {k}")
    evaluated = np.zeros(length, dtype=bool)
    evaluated[seed] = True
    tau_seed = float(scores[seed].min())
    fallback = policy.fallback_threshold is not None and fallback_value is not None and fallback_value > policy.fallback_threshold
    full_refresh = bool(policy.name == "full" or (policy.refresh_interval and step % policy.refresh_interval == 0) or fallback)
    current_max = block_max_f32(scores, block_size)
    if policy.risk_model == "last_max":
        risk = last_max.astype(np.float64) + policy.gamma + policy.age_slope * age
    elif policy.risk_model == "ema":
        risk = ema.astype(np.float64) + policy.volatility_lambda * volatility + policy.gamma + policy.age_slope * age
    else:
        raise ValueError(f"unknown risk model: {policy.risk_model}")
    if policy.order == "oracle_current":
        order = np.asarray(sorted(range(blocks), key=lambda b: (-current_max[b], b)), dtype=np.int64)
    else:
        order = order_blocks(policy, risk)

    threshold = tau_seed
    heap: list | None = None
    if policy.dynamic_threshold:
        # min-heap on (score, -key): the worst kept item is the smallest score,
        # and among equal scores the larger key.
        heap = [(float(scores[key]), -int(key)) for key in seed]
        heapq.heapify(heap)
    refreshed = np.zeros(blocks, dtype=bool)
    skipped = np.zeros(blocks, dtype=bool)
    new_block = np.zeros(blocks, dtype=bool)
    if previous_length < length:
        new_block[previous_length // block_size :] = True
    recent = np.zeros(blocks, dtype=bool)
    if policy.recent_window:
        recent[max(0, length - policy.recent_window) // block_size :] = True
    if wave < 1:
        raise ValueError("wave must be >= 1")
    for start in range(0, order.size, wave):
        fresh_keys = []
        for b in order[start : start + wave]:
            b = int(b)
            lo, hi = b * block_size, min(length, (b + 1) * block_size)
            forced = (
                full_refresh
                or new_block[b]
                or recent[b]
                or (policy.age_cap is not None and age[b] >= policy.age_cap)
                or cold[b] < policy.cold_streak
            )
            if not forced and risk[b] < threshold:
                skipped[b] = True
                continue
            unseen = lo + np.flatnonzero(~evaluated[lo:hi])
            evaluated[lo:hi] = True
            refreshed[b] = True
            if unseen.size:
                fresh_keys.append(unseen)
        if heap is not None and fresh_keys:
            unseen = np.concatenate(fresh_keys)
            floor = heap[0][0]
            for key in unseen[scores[unseen] >= floor]:
                item = (float(scores[key]), -int(key))
                if item > heap[0]:
                    heapq.heapreplace(heap, item)
            threshold = heap[0][0]

    scored = np.flatnonzero(evaluated)
    if heap is None:
        if scored.size < k:
            raise RuntimeError(f"policy scored {scored.size} keys, fewer than K={k}")
        approximate = scored[stable_topk(scores[scored], k)]
    else:
        approximate = np.asarray([-item[1] for item in sorted(heap, reverse=True)], dtype=np.int64)
    approx_mask = np.zeros(length, dtype=bool)
    approx_mask[approximate] = True
    base_mask = np.zeros(length, dtype=bool)
    base_mask[baseline] = True
    retained = int(base_mask[approximate].sum())

    new_last = last_max.copy()
    new_ema = ema.copy()
    new_vol = volatility.copy()
    new_age = np.minimum(age.astype(np.int32) + 1, np.iinfo(np.int16).max).astype(np.int16)
    for b in np.flatnonzero(refreshed):
        seen = float(current_max[b])
        mean = float(ema[b]) if np.isfinite(ema[b]) else seen
        new_last[b] = seen
        new_ema[b] = policy.ema_alpha * seen + (1.0 - policy.ema_alpha) * mean
        new_vol[b] = policy.ema_alpha * abs(seen - mean) + (1.0 - policy.ema_alpha) * volatility[b]
        new_age[b] = 0
    if history_mode == "teacher":
        new_last = current_max.copy()
        new_ema = current_max.copy()
        new_vol[:] = 0.0
        new_age[:] = 0
    hot = np.zeros(blocks, dtype=bool)
    hot[(baseline if history_mode == "teacher" else approximate) // block_size] = True
    next_cold = np.where(hot, 0, np.minimum(cold.astype(np.int32) + 1, 32767)).astype(np.int16)
    next_state = ApproxState(approximate, baseline, new_last, new_ema, new_vol, new_age, next_cold)

    newly_hot = np.setdiff1d(baseline, state.baseline_topk)
    newly_missed = int((~approx_mask[newly_hot]).sum()) if newly_hot.size else 0
    missed_rank = np.flatnonzero(~approx_mask[baseline]) + 1
    seed_blocks = np.unique(seed // block_size)
    meta_bpb = metadata_bytes_per_block(policy)
    meta = blocks * meta_bpb
    metrics: dict[str, Any] = {
        "step": step,
        "context_length": length,
        "history_mode": history_mode,
        "policy": policy.name,
        "gamma": policy.gamma,
        "k": k,
        "block_size": block_size,
        "qk_scored": int(scored.size),
        "qk_reduction": float(1.0 - scored.size / length),
        "exact_match": bool(np.array_equal(np.sort(approximate), np.sort(baseline))),
        "recall": float(retained / k),
    }
    for count in (128, 256, 512, 1024, 2048):
        metrics[f"top{count}_recall"] = _retention(approximate, baseline, count)
    metrics.update({
        "index_mass_ratio": _mass_ratio(scores, approximate, baseline),
        "newly_hot_count": int(newly_hot.size),
        "newly_hot_missed": newly_missed,
        "newly_hot_miss_rate": float(newly_missed / newly_hot.size) if newly_hot.size else 0.0,
        "missed_count": int(missed_rank.size),
        "worst_missed_rank": int(missed_rank.min()) if missed_rank.size else 0,
        "tau_seed": tau_seed,
        "tau_final": float(np.min(scores[approximate])),
        "full_refresh": full_refresh,
        "fallback": bool(fallback),
        "blocks_refreshed": int(refreshed.sum()),
        "blocks_skipped": int(skipped.sum()),
        "seed_blocks_touched": int(seed_blocks.size),
        "seed_block_fraction": float(seed_blocks.size / blocks),
        "metadata_bytes_per_block": meta_bpb,
        "metadata_bytes": meta,
        "ideal_bf16_bytes": int(scored.size * 256 + meta),
        "ideal_fp8_bytes": int(scored.size * 128 + meta),
        "net_bf16_reduction": float(1.0 - (scored.size * 256 + meta) / (length * 256)),
        "net_fp8_reduction": float(1.0 - (scored.size * 128 + meta) / (length * 128)),
    })
    for physical in (16, 32, 64, 128):
        touched = np.unique(scored // physical).size
        total = (length + physical - 1) // physical
        metrics[f"physical_b{physical}_blocks"] = int(touched)
        metrics[f"physical_b{physical}_reduction"] = float(1.0 - touched / total)
    for entries in (0, 256, 512, 1024, 2048):
        uncached = evaluated.copy()
        uncached[seed[: min(entries, seed.size)]] = False
        hbm = int(uncached.sum())
        metrics[f"cache{entries}_hbm_keys"] = hbm
        metrics[f"cache{entries}_net_bf16_reduction"] = float(1.0 - (hbm * 256 + meta) / (length * 256))
    details = {
        "approximate": approximate,
        "baseline": baseline,
        "evaluated": scored,
        "seed": seed.copy(),
        "refreshed_blocks": np.flatnonzero(refreshed).astype(np.int32),
        "skipped_blocks": np.flatnonzero(skipped).astype(np.int32),
        "missed_ranks": missed_rank.astype(np.int32),
    }
    return next_state, metrics, details
