"""CPU restatement of the temporal pruning replay (test oracle).

Reference: replay.py:114-400 (ReplayResult, _block_slices, _block_max,
_scan_order, _run_filter / _compiled_filter, replay_transition) and
replay.py:476-627 (replay_trace).

One extension: ``wave``.  The reference refreshes the running top-K threshold
after every kept block; a GPU processes a wave of blocks at once.  With
``wave = W`` the scan order is cut into consecutive groups of W blocks; every
block of a group is pruned or kept against the threshold in force at the start
of the group, and the threshold is refreshed after the group.  ``wave = 1``
reproduces the reference schedule exactly.
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass

import numpy as np

from .topk import stable_topk

METHODS = ("full", "static", "static_hot_first", "dynamic", "oracle")
SCAN_ORDERS = ("address", "previous_hot", "upper_hot", "oracle_current")


@dataclass(frozen=True)
class ReplayResult:
    """Reference: replay.py:114-142 (same fields, same order)."""

    method: str
    scan_order: str
    step: int
    layer: int
    workload: str
    prompt_id: str
    context_length: int
    k: int
    block_size: int
    gamma_sigma: float
    gamma: float
    tau_seed: float
    tau_final: float
    threshold_ratio: float
    threshold_gap: float
    qk_scored: int
    qk_reduction: float
    blocks_pruned: int
    block_pruning_rate: float
    false_cold_blocks: int
    false_cold_rate: float
    recall: float
    exact_match: bool
    discovery_fraction: float
    key_bytes: int
    metadata_bytes: int
    net_byte_reduction: float


def block_maxima(values: np.ndarray, block_size: int) -> np.ndarray:
    """Max of each block [b*bs, min(n, (b+1)*bs)).  Reference: replay.py:145-150."""

    values = np.asarray(values, dtype=np.float64)
    blocks = math.ceil(values.size / block_size)
    out = np.empty(blocks)
    for b in range(blocks):
        out[b] = values[b * block_size : (b + 1) * block_size].max()
    return out


def block_scan_order(name: str, upper: np.ndarray, current_max: np.ndarray, previous_hot: np.ndarray) -> np.ndarray:
    """Block visiting order.  Reference: replay.py:153-169.

    address: 0..n-1; previous_hot: hot blocks first, then larger upper bound,
    then lower address; upper_hot: larger upper bound, then address;
    oracle_current: larger current block max, then address.
    """

    n = upper.size
    ids = list(range(n))
    if name == "address":
        return np.arange(n)
    if name == "previous_hot":
        ids.sort(key=lambda b: (not previous_hot[b], -upper[b], b))
    elif name == "upper_hot":
        ids.sort(key=lambda b: (-upper[b], b))
    elif name == "oracle_current":
        ids.sort(key=lambda b: (-current_max[b], b))
    else:
        raise ValueError(f"unknown scan order: {name}")
    return np.asarray(ids, dtype=np.int64)


@dataclass
class FilterTrace:
    """Outcome of one pruning scan."""

    evaluated: np.ndarray  # bool [L]
    kept: np.ndarray  # bool [blocks]: scanned and not pruned
    pruned: list  # block ids in scan order
    scored: int
    positions: np.ndarray  # evaluation position (1-based), L for never evaluated
    threshold_final: float


def run_filter(
    current: np.ndarray,
    seed: np.ndarray,
    k: int,
    block_size: int,
    upper: np.ndarray,
    order: np.ndarray,
    *,
    dynamic: bool,
    fixed_threshold: float,
    wave: int = 1,
) -> FilterTrace:
    """Seeded block scan with pruning ``upper[b] < threshold``.

    Reference: replay.py:172-222 and the equivalent compiled path replay.py:47-109.
    Seeds (previous top-K) are scored first; kept blocks score their unseen
    keys in address order; the dynamic threshold is the k-th largest score
    among evaluated keys, refreshed after every group of ``wave`` blocks.
    """

    length = current.size
    evaluated = np.zeros(length, dtype=bool)
    positions = np.full(length, length, dtype=np.int64)
    scored = 0
    for key in seed:
        key = int(key)
        if key < length and not evaluated[key]:
            evaluated[key] = True
            scored += 1
            positions[key] = scored
    threshold = float(fixed_threshold)
    kept = np.zeros(upper.size, dtype=bool)
    pruned: list[int] = []
    for start in range(0, order.size, wave):
        group = order[start : start + wave]
        decisions = [upper[b] < threshold for b in group]
        for b, prune in zip(group, decisions):
            b = int(b)
            if prune:
                pruned.append(b)
                continue
            kept[b] = True
            lo, hi = b * block_size, min(length, (b + 1) * block_size)
            for key in range(lo, hi):
                if not evaluated[key]:
                    evaluated[key] = True
                    scored += 1
                    positions[key] = scored
        if dynamic and np.count_nonzero(evaluated) >= k:
            threshold = float(np.partition(current[evaluated], -k)[-k])
    return FilterTrace(evaluated, kept, pruned, scored, positions, threshold)


def transition_setup(previous: np.ndarray, current: np.ndarray, block_size: int):
    """Block maxima of both steps and the score drift sigma.  Reference: replay.py:252-258."""

    current_max = block_maxima(current, block_size)
    previous_max = np.full(current_max.size, -np.inf)
    prev_blocks = block_maxima(previous, block_size)
    previous_max[: prev_blocks.size] = prev_blocks
    sigma = float(np.std(current[: previous.size] - previous))
    return current_max, previous_max, sigma


def upper_bounds(previous_max: np.ndarray, gamma: float, previous_length: int, current_length: int, block_size: int) -> np.ndarray:
    """prev block max + gamma; blocks holding new keys are never pruned.  Reference: replay.py:261-266."""

    upper = previous_max + gamma
    if previous_length < current_length:
        upper[previous_length // block_size :] = np.inf
    return upper


def method_schedule(method: str, requested_order: str) -> tuple[str, bool, bool]:
    """(order, dynamic threshold, bound is the oracle current max).  Reference: replay.py:274-297,319-359."""

    if method == "static":
        return "address", False, False
    if method == "static_hot_first":
        return "previous_hot", False, False
    if method == "dynamic":
        return requested_order, True, False
    if method == "oracle":
        return "oracle_current", True, True
    raise ValueError(f"unknown method: {method}")


def replay_transition(
    previous,
    current,
    *,
    k: int,
    block_size: int,
    gamma_sigma: float,
    method: str,
    scan_order: str = "address",
    step: int = 0,
    layer: int = 0,
    workload: str = "synthetic",
    prompt_id: str = "0",
    key_bytes: int = 256,
    metadata_bytes_per_block: int = 8,
    wave: int = 1,
    absolute_gamma: float | None = None,
    previous_topk: np.ndarray | None = None,
    true_topk: np.ndarray | None = None,
    return_trace: bool = False,
    sigma: float | None = None,
):
    """Replay one decode transition.  Reference: replay.py:225-400.

    ``sigma`` overrides the score-drift estimate, as the trace sweep's block
    cache does (replay.py:482-483 computes it on the trace's float32 rows).
    """

    previous = np.asarray(previous, dtype=np.float64)
    current = np.asarray(current, dtype=np.float64)
    if previous.ndim != 1 or current.ndim != 1 or previous.size > current.size:
        raise ValueError("expected 1-D scores with previous length <= current length")
    if not 0 < k <= previous.size:
        raise ValueError("k must fit the previous step so it can seed replay")
    current_max, previous_max, own_sigma = transition_setup(previous, current, block_size)
    sigma = own_sigma if sigma is None else float(sigma)
    gamma = gamma_sigma * sigma if absolute_gamma is None else float(absolute_gamma)
    upper = upper_bounds(previous_max, gamma, previous.size, current.size, block_size)
    seed = stable_topk(previous, k) if previous_topk is None else np.asarray(previous_topk)
    truth = stable_topk(current, k) if true_topk is None else np.asarray(true_topk)
    tau_seed = float(np.min(current[seed]))
    tau_final = float(np.min(current[truth]))
    blocks = current_max.size
    trace = None
    if method == "full":
        qk_scored = current.size
        pruned_count = 0
        pruned_true = 0
        true_evaluated = k
        discovery = 1.0
        order_name = scan_order
    else:
        order_name, dynamic, oracle_bound = method_schedule(method, scan_order)
        bound = current_max if oracle_bound else upper
        hot = np.zeros(blocks, dtype=bool)
        hot[np.minimum(seed // block_size, blocks - 1)] = True
        order = block_scan_order(order_name, bound, current_max, hot)
        trace = run_filter(current, seed, k, block_size, bound, order, dynamic=dynamic, fixed_threshold=tau_seed, wave=wave)
        qk_scored = trace.scored
        pruned_count = len(trace.pruned)
        truth_blocks = np.zeros(blocks, dtype=bool)
        truth_blocks[truth // block_size] = True
        pruned_true = int(truth_blocks[np.asarray(trace.pruned, dtype=np.int64)].sum()) if trace.pruned else 0
        true_evaluated = int(trace.evaluated[truth].sum())
        discovery = float(np.max(trace.positions[truth], initial=0) / current.size)
    metadata_bytes = blocks * metadata_bytes_per_block
    bytes_read = qk_scored * key_bytes + metadata_bytes
    result = ReplayResult(
        method=method,
        scan_order=order_name,
        step=step,
        layer=layer,
        workload=workload,
        prompt_id=prompt_id,
        context_length=current.size,
        k=k,
        block_size=block_size,
        gamma_sigma=gamma_sigma,
        gamma=gamma,
        tau_seed=tau_seed,
        tau_final=tau_final,
        threshold_ratio=tau_seed / tau_final if tau_final != 0 else math.nan,
        threshold_gap=tau_final - tau_seed,
        qk_scored=qk_scored,
        qk_reduction=1.0 - qk_scored / current.size,
        blocks_pruned=pruned_count,
        block_pruning_rate=pruned_count / blocks,
        false_cold_blocks=pruned_true,
        false_cold_rate=pruned_true / pruned_count if pruned_count else 0.0,
        recall=true_evaluated / k,
        exact_match=true_evaluated == k,
        discovery_fraction=discovery,
        key_bytes=key_bytes,
        metadata_bytes=metadata_bytes,
        net_byte_reduction=1.0 - bytes_read / (current.size * key_bytes),
    )
    return (result, trace) if return_trace else result


SWEEP_VARIANTS = (
    ("static", "address"),
    ("static_hot_first", "previous_hot"),
    ("dynamic", "address"),
    ("dynamic", "previous_hot"),
    ("dynamic", "upper_hot"),
    ("dynamic", "oracle_current"),
)
CALIBRATED_VARIANTS = SWEEP_VARIANTS[:5]


def replay_trace_rows(
    rows: list,
    *,
    k_values,
    block_sizes,
    gamma_sigma_values,
    key_bytes: int = 256,
    metadata_bytes_per_block: int = 8,
    absolute_margins: dict | None = None,
    layer: int = 0,
    workload: str = "synthetic",
    prompt_id: str = "0",
    wave: int = 1,
) -> list[dict]:
    """Per-transition sweep over a trace given as score rows.  Reference: replay.py:476-591."""

    out: list[dict] = []
    for step in range(1, len(rows)):
        previous = np.asarray(rows[step - 1], dtype=np.float64)
        current = np.asarray(rows[step], dtype=np.float64)
        # The drift is taken in the rows' own precision (float32 for a trace).
        row_prev = np.asarray(rows[step - 1])
        sigma = float(np.std(np.asarray(rows[step])[: row_prev.size] - row_prev))
        for k in k_values:
            if k > previous.size:
                continue
            seed = stable_topk(previous, k)
            truth = stable_topk(current, k)
            for bs in block_sizes:
                common = dict(
                    k=k, block_size=bs, step=step, layer=layer, workload=workload, prompt_id=prompt_id,
                    key_bytes=key_bytes, metadata_bytes_per_block=metadata_bytes_per_block,
                    previous_topk=seed, true_topk=truth, wave=wave, sigma=sigma,
                )
                for method, order in (("full", "address"), ("oracle", "oracle_current")):
                    out.append(asdict(replay_transition(previous, current, gamma_sigma=0.0, method=method, scan_order=order, **common)))
                for gs in gamma_sigma_values:
                    for method, order in SWEEP_VARIANTS:
                        out.append(asdict(replay_transition(previous, current, gamma_sigma=gs, method=method, scan_order=order, **common)))
                if absolute_margins and bs in absolute_margins:
                    for method, order in CALIBRATED_VARIANTS:
                        out.append(asdict(replay_transition(
                            previous, current, gamma_sigma=-1.0, method=method, scan_order=order,
                            absolute_gamma=float(absolute_margins[bs]), **common,
                        )))
    return out


def aggregate_rows(rows: list[dict]):
    """Group and summarise per-transition rows.  Reference: replay.py:592-627."""

    import pandas as pd

    frame = pd.DataFrame(rows)
    if frame.empty:
        return frame
    keys = ["layer", "workload", "prompt_id", "k", "block_size", "gamma_sigma", "method", "scan_order"]
    return frame.groupby(keys, as_index=False).agg(
        transition_count=("step", "count"),
        context_length=("context_length", "median"),
        gamma=("gamma", "median"),
        tau_seed=("tau_seed", "median"),
        tau_final=("tau_final", "median"),
        threshold_ratio=("threshold_ratio", "median"),
        threshold_gap=("threshold_gap", "median"),
        qk_scored=("qk_scored", "median"),
        qk_reduction=("qk_reduction", "median"),
        qk_reduction_p5=("qk_reduction", lambda x: x.quantile(0.05)),
        qk_reduction_p95=("qk_reduction", lambda x: x.quantile(0.95)),
        blocks_pruned=("blocks_pruned", "median"),
        block_pruning_rate=("block_pruning_rate", "median"),
        false_cold_blocks=("false_cold_blocks", "sum"),
        false_cold_rate=("false_cold_rate", "mean"),
        recall=("recall", "mean"),
        exact_match=("exact_match", "mean"),
        discovery_fraction=("discovery_fraction", "median"),
        key_bytes=("key_bytes", "first"),
        metadata_bytes=("metadata_bytes", "median"),
        net_byte_reduction=("net_byte_reduction", "median"),
    )


# ---------------------------------------------------------------------------
# Per-transition statistics tables (reference replay.py:403-474, the inputs of
# the analyze command's temporal_stats.csv and block_stats.csv).
# ---------------------------------------------------------------------------
def pearson(x, y) -> float:
    """Reference metrics.py:40-47: float64 correlation, NaN for fewer than two
    values or a constant vector."""

    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    if x.size != y.size or x.size < 2 or np.std(x) == 0 or np.std(y) == 0:
        return math.nan
    xc = x - x.mean()
    yc = y - y.mean()
    return float(np.clip(np.dot(xc, yc) / math.sqrt(np.dot(xc, xc) * np.dot(yc, yc)), -1.0, 1.0))


def average_ranks(x) -> np.ndarray:
    """0-based ascending ranks, tied values sharing the mean of their
    positions (reference metrics.py:50-61)."""

    x = np.asarray(x)
    order = np.argsort(x, kind="stable")
    ranks = np.empty(x.size, dtype=np.float64)
    sx = x[order]
    # run boundaries of equal values in ascending order
    cuts = np.flatnonzero(np.concatenate(([True], sx[1:] != sx[:-1], [True])))
    for start, end in zip(cuts[:-1], cuts[1:]):
        ranks[order[start:end]] = 0.5 * (start + end - 1)
    return ranks


def spearman(x, y) -> float:
    """Reference metrics.py:64-69."""

    return pearson(average_ranks(x), average_ranks(y))


def temporal_stats_rows(rows: list[np.ndarray], k_values, *, layer=0, workload="", prompt_id="") -> list[dict]:
    """One record per (transition, k <= common length): score correlations,
    the score drift and the top-k overlap of consecutive rows (reference
    replay.py:403-428)."""

    out = []
    for step in range(1, len(rows)):
        prev = np.asarray(rows[step - 1], dtype=np.float32)
        cur = np.asarray(rows[step], dtype=np.float32)
        n = min(prev.size, cur.size)
        p, c = prev[:n], cur[:n]
        delta = c - p  # float32, as the reference subtracts float32 rows
        base = {
            "step": step, "layer": layer, "workload": workload, "prompt_id": prompt_id,
            "context_length": cur.size,
            "score_pearson": pearson(p, c),
            "score_spearman": spearman(p, c),
            "delta_mean": float(np.mean(delta)),
            "delta_std": float(np.std(delta)),
            "delta_p99_abs": float(np.percentile(np.abs(delta), 99)),
        }
        for k in k_values:
            if k > n:
                continue
            a = set(stable_topk(p, k).tolist())
            b = stable_topk(c, k)
            overlap = sum(1 for i in b.tolist() if i in a) / b.size
            out.append({**base, "k": k, "topk_overlap": overlap})
    return out


def block_temporal_stats_rows(rows: list[np.ndarray], block_sizes, k_values, *, layer=0, workload="",
                              prompt_id="") -> list[dict]:
    """One record per (transition, block size, k <= common length): the
    drift of the block maxima and the fraction of blocks cold (block maximum
    below the current k-th largest score) for at least 1, 2, 4 and 8
    consecutive steps (reference replay.py:431-474)."""

    out = []
    streak: dict[tuple[int, int], np.ndarray] = {}
    for step in range(1, len(rows)):
        prev = np.asarray(rows[step - 1], dtype=np.float32)
        cur = np.asarray(rows[step], dtype=np.float32)
        n = min(prev.size, cur.size)
        for bs in block_sizes:
            pm = block_maxima(prev[:n], bs)
            cm = block_maxima(cur[:n], bs)
            for k in k_values:
                if k > n:
                    continue
                threshold = float(np.sort(cur[:n])[n - k])
                state = streak.setdefault((bs, k), np.zeros(0, dtype=np.int32))
                if state.size < cm.size:
                    state = np.concatenate((state, np.zeros(cm.size - state.size, dtype=np.int32)))
                cold = cm < threshold
                state[: cm.size] = np.where(cold, state[: cm.size] + 1, 0)
                streak[(bs, k)] = state
                s = state[: cm.size]
                delta = cm - pm
                out.append({
                    "step": step, "layer": layer, "workload": workload, "prompt_id": prompt_id,
                    "context_length": cur.size, "k": k, "block_size": bs, "topk_threshold": threshold,
                    "delta_max_mean": float(np.mean(delta)),
                    "delta_max_p5": float(np.percentile(delta, 5)),
                    "delta_max_median": float(np.median(delta)),
                    "delta_max_p95": float(np.percentile(delta, 95)),
                    "cold_fraction_1": float(np.mean(s >= 1)),
                    "cold_fraction_2": float(np.mean(s >= 2)),
                    "cold_fraction_4": float(np.mean(s >= 4)),
                    "cold_fraction_8": float(np.mean(s >= 8)),
                })
    return out
