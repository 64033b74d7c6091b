"""Temporal-pruning replay over recorded score traces, on the GPU.

The reference's analysis (reference replay.py:225-400 ``replay_transition``,
:476-627 ``replay_trace``) replays each decode transition of a
:class:`~dsa_amd.trace.ScoreTrace` through the pruning filter: seeds are the
previous step's stable top-k, block b is pruned iff
``previous block max + gamma < threshold``, with blocks holding new keys
never pruned, and the threshold is the seeds' minimum (static) or the k-th
largest score evaluated so far (dynamic).  Here every filter runs in the HIP
temporal kernels (``dsa_temporal_replay_step``), with the trace row as the
score source, batched over the gamma values of a transition.  The host
derives the reference's result fields from the kernels' outputs: refreshed
blocks, keys scored, scan order and the scores of the evaluated keys.

Methods and orders keep the reference's names: ``full``; ``static``
(address order); ``static_hot_first`` (previous-hot order); ``dynamic`` with
``address`` / ``previous_hot`` / ``upper_hot``; and ``oracle`` /
``oracle_current`` (the current block maxima as the bound and order).  The
drift sigma of a transition is numpy's float32 ``std`` of the rows'
difference, as the reference computes it.  ``wave`` > 1 refreshes the dynamic
threshold after every ``wave`` blocks instead of every block (the
reference's schedule is ``wave=1``).
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass

import numpy as np
import torch

from . import _lib
from .metrics import topk as device_topk
from .temporal import block_max
from .trace import ScoreTrace

_ORDER_CODES = {"address": 0, "previous_hot": 1, "upper_hot": 2, "oracle_current": 3}
SWEEP_VARIANTS = (
    ("static", "address"),
    ("static_hot_first", "previous_hot"),
    ("dynamic", "address"),
    ("dynamic", "previous_hot"),
    ("dynamic", "upper_hot"),
    ("dynamic", "oracle_current"),
)
CALIBRATED_VARIANTS = SWEEP_VARIANTS[:5]



@dataclass(frozen=True)
class ReplayResult:
    """One replayed transition (reference replay.py:114-142; same fields, same order)."""

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


def _workspace(device, stream, rows, length, k, block_size) -> torch.Tensor:
    need = int(_lib.query("dsa_temporal_workspace_bytes", rows, length, k, block_size))
    return _lib.workspace("temporal", device, stream, need, zeroed=False)


def _schedule(method: str, order: str) -> tuple[str, bool, bool]:
    """(order, dynamic threshold, current maxima as the bound)."""

    if method == "static":
        return "address", False, False
    if method == "static_hot_first":
        return "previous_hot", False, False
    if method == "dynamic":
        return order, True, False
    if method == "oracle":
        return "oracle_current", True, True
    raise ValueError(f"unknown method: {method}")


class _Transition:
    """GPU-resident inputs of one transition for one (k, block size)."""

    def __init__(self, previous: torch.Tensor, current: torch.Tensor, k: int, block_size: int,
                 seed: torch.Tensor, truth: torch.Tensor):
        self.previous, self.current = previous, current
        self.k, self.bs = k, block_size
        self.length = current.numel()
        self.prev_length = previous.numel()
        self.blocks = -(-self.length // block_size)
        self.prev_max = block_max(previous.reshape(1, -1), block_size)
        self.cur_max = block_max(current.reshape(1, -1), block_size)
        self.seed = seed
        host = current.cpu().numpy().astype(np.float64)
        self.host = host
        self.seed_h = seed.cpu().numpy()
        self.truth_h = truth.cpu().numpy()
        self.tau_seed = float(np.min(host[self.seed_h]))
        self.tau_final = float(np.min(host[self.truth_h]))
        self.truth_blocks = np.zeros(self.blocks, dtype=bool)
        self.truth_blocks[self.truth_h // block_size] = True

    def run(self, gammas: list[float], order: str, dynamic: bool, oracle: bool, wave: int):
        """The filter for every gamma (one row each): (kept [G, nb], qk [G],
        evaluated-key mask [G, L], scan order [G, nb])."""

        rows = len(gammas)
        dev = self.current.device
        bound = self.cur_max if oracle else self.prev_max
        prev_length = self.length if oracle else self.prev_length
        code = _ORDER_CODES[order]
        key_rows = self.cur_max.expand(rows, -1).contiguous() if order == "oracle_current" else None
        # the oracle's bound is the current maxima themselves: its gamma is reported, not applied
        g = torch.tensor([0.0] * rows if oracle else gammas, dtype=torch.float64, device=dev)
        bound_rows = bound.expand(rows, -1).contiguous()
        seeds = self.seed.reshape(1, -1).expand(rows, -1).contiguous()
        scores = torch.empty((rows, self.length), device=dev, dtype=torch.float32)
        kept = torch.empty((rows, self.blocks), device=dev, dtype=torch.uint8)
        order_out = torch.empty((rows, self.blocks), device=dev, dtype=torch.int32)
        top = torch.empty((rows, self.k), device=dev, dtype=torch.int64)
        qk = torch.empty(rows, device=dev, dtype=torch.int32)
        ws = _workspace(dev, _lib.stream_of(self.current), rows, self.length, self.k, self.bs)
        _lib.call(
            "dsa_temporal_replay_step", _lib.ptr(self.current), 0, _lib.ptr(bound_rows), prev_length,
            _lib.ptr(seeds), _lib.ptr(g), _lib.ptr(key_rows), _lib.ptr(scores), _lib.ptr(kept), _lib.ptr(order_out), _lib.ptr(top),
            _lib.ptr(qk), rows, self.length, self.k, self.bs, code, wave if dynamic else 0, _lib.ptr(ws),
            ws.numel(), _lib.stream_of(self.current),
        )
        return (kept.cpu().numpy().astype(bool), qk.cpu().numpy(), np.isfinite(scores.cpu().numpy()),
                order_out.cpu().numpy())

    def discovery(self, evaluated: np.ndarray, kept: np.ndarray, order: np.ndarray) -> float:
        """max over the true top-k of its evaluation position / L (replay.py:209-216):
        seeds count first in seed order, then the unseen keys of kept blocks in
        scan order, address order within a block."""

        length, bs = self.length, self.bs
        position = np.full(length, length, dtype=np.int64)
        seeds = self.seed_h[self.seed_h < length]
        position[seeds] = np.arange(1, seeds.size + 1)
        is_seed = np.zeros(length, dtype=bool)
        is_seed[seeds] = True
        done = seeds.size
        for b in order[kept[order]].tolist():
            keys = np.arange(b * bs, min(length, (b + 1) * bs))
            fresh = keys[~is_seed[keys]]
            position[fresh] = done + 1 + np.arange(fresh.size)
            done += fresh.size
        return float(np.max(position[self.truth_h], initial=0) / length)


def _result(t: _Transition, *, method, order_name, gamma_sigma, gamma, qk_scored, pruned, false_cold, true_eval,
            discovery, step, layer, workload, prompt_id, key_bytes, metadata_bytes_per_block) -> ReplayResult:
    metadata_bytes = t.blocks * metadata_bytes_per_block
    bytes_read = qk_scored * key_bytes + metadata_bytes
    return ReplayResult(
        method=method, scan_order=order_name, step=step, layer=layer, workload=workload, prompt_id=prompt_id,
        context_length=t.length, k=t.k, block_size=t.bs, gamma_sigma=gamma_sigma, gamma=gamma,
        tau_seed=t.tau_seed, tau_final=t.tau_final,
        threshold_ratio=t.tau_seed / t.tau_final if t.tau_final != 0 else math.nan,
        threshold_gap=t.tau_final - t.tau_seed, qk_scored=int(qk_scored), qk_reduction=1.0 - qk_scored / t.length,
        blocks_pruned=int(pruned), block_pruning_rate=pruned / t.blocks, false_cold_blocks=int(false_cold),
        false_cold_rate=false_cold / pruned if pruned else 0.0, recall=true_eval / t.k, exact_match=true_eval == t.k,
        discovery_fraction=discovery, key_bytes=key_bytes, metadata_bytes=metadata_bytes,
        net_byte_reduction=1.0 - bytes_read / (t.length * key_bytes),
    )


def _replay_variants(t: _Transition, variants: list[tuple[str, str, float, float]], *, wave: int,
                     **info) -> list[ReplayResult]:
    """Replay (method, order, gamma_sigma, gamma) variants of one transition,
    one kernel call per (method, order) batched over its gammas."""

    out: dict[int, ReplayResult] = {}
    groups: dict[tuple[str, str], list[int]] = {}
    for i, (method, order, _, _) in enumerate(variants):
        if method == "full":
            truth_eval = t.k
            out[i] = _result(t, method="full", order_name=order, gamma_sigma=variants[i][2], gamma=variants[i][3],
                             qk_scored=t.length, pruned=0, false_cold=0, true_eval=truth_eval, discovery=1.0, **info)
            continue
        groups.setdefault((method, order), []).append(i)
    for (method, order), idx in groups.items():
        order_name, dynamic, oracle = _schedule(method, order)
        gammas = [variants[i][3] for i in idx]
        kept, qk, evaluated, scan = t.run(gammas, order_name, dynamic, oracle, wave)
        for row, i in enumerate(idx):
            pruned_blocks = ~kept[row]
            pruned = int(pruned_blocks.sum())
            false_cold = int((t.truth_blocks & pruned_blocks).sum())
            true_eval = int(evaluated[row][t.truth_h].sum())
            out[i] = _result(t, method=method, order_name=order_name, gamma_sigma=variants[i][2], gamma=variants[i][3],
                             qk_scored=int(qk[row]), pruned=pruned, false_cold=false_cold, true_eval=true_eval,
                             discovery=t.discovery(evaluated[row], kept[row], scan[row]), **info)
    return [out[i] for i in range(len(variants))]


def replay_transition(previous, current, *, k: int, block_size: int, gamma_sigma: float, method: str,
                      scan_order: str = "address", step: int = 0, layer: int = 0, workload: str = "synthetic",
                      prompt_id: str = "0", key_bytes: int = 256, metadata_bytes_per_block: int = 8,
                      absolute_gamma: float | None = None, wave: int = 1) -> ReplayResult:
    """Replay one decode transition (reference replay.py:225-400) on the GPU.
    ``previous`` / ``current`` are the two steps' score rows (numpy or GPU)."""

    _lib.load()
    dev = torch.device("cuda", torch.cuda.current_device())
    prev = torch.as_tensor(np.asarray(previous, dtype=np.float32) if not isinstance(previous, torch.Tensor) else previous,
                           device=dev).to(torch.float32).contiguous()
    cur = torch.as_tensor(np.asarray(current, dtype=np.float32) if not isinstance(current, torch.Tensor) else current,
                          device=dev).to(torch.float32).contiguous()
    if prev.ndim != 1 or cur.ndim != 1 or prev.numel() > cur.numel():
        raise ValueError("expected 1-D scores with previous length <= current length")
    if not 0 < k <= prev.numel():
        raise ValueError("k must fit the previous step so it can seed replay")
    ph, ch = prev.cpu().numpy(), cur.cpu().numpy()
    sigma = float(np.std(ch[: ph.size] - ph))
    gamma = gamma_sigma * sigma if absolute_gamma is None else float(absolute_gamma)
    seed = device_topk(prev.reshape(1, -1), k, sorted=True)[0]
    truth = device_topk(cur.reshape(1, -1), k, sorted=True)[0]
    t = _Transition(prev, cur, k, block_size, seed, truth)
    return _replay_variants(t, [(method, scan_order, gamma_sigma, gamma)], wave=wave, step=step, layer=layer,
                            workload=workload, prompt_id=prompt_id, key_bytes=key_bytes,
                            metadata_bytes_per_block=metadata_bytes_per_block)[0]


def replay_trace_rows(trace: ScoreTrace, *, k_values, block_sizes, gamma_sigma_values, key_bytes: int = 256,
                      metadata_bytes_per_block: int = 8, absolute_margins: dict | None = None,
                      wave: int = 1) -> list[dict]:
    """Per-transition rows of the reference's sweep (replay.py:476-591), in its order."""

    _lib.load()
    dev = torch.device("cuda", torch.cuda.current_device())
    info = dict(layer=trace.layer, workload=trace.workload, prompt_id=trace.prompt_id, key_bytes=key_bytes,
                metadata_bytes_per_block=metadata_bytes_per_block)
    rows: list[dict] = []
    for step in range(1, trace.scores.shape[0]):
        ph, ch = trace.row(step - 1), trace.row(step)
        sigma = float(np.std(ch[: ph.size] - ph))
        prev = torch.from_numpy(ph).to(dev)
        cur = torch.from_numpy(ch).to(dev)
        for k in k_values:
            if k > ph.size:
                continue
            seed = device_topk(prev.reshape(1, -1), k, sorted=True)[0]
            truth = device_topk(cur.reshape(1, -1), k, sorted=True)[0]
            for bs in block_sizes:
                t = _Transition(prev, cur, k, bs, seed, truth)
                variants = [("full", "address", 0.0, 0.0), ("oracle", "oracle_current", 0.0, 0.0)]
                for gs in gamma_sigma_values:
                    variants += [(m, o, gs, gs * sigma) for m, o in SWEEP_VARIANTS]
                if absolute_margins and bs in absolute_margins:
                    variants += [(m, o, -1.0, float(absolute_margins[bs])) for m, o in CALIBRATED_VARIANTS]
                replayed = _replay_variants(t, variants, wave=wave, step=step, **info)
                rows.extend(asdict(r) for r in replayed)
    return rows


def replay_trace(trace: ScoreTrace, *, k_values, block_sizes, gamma_sigma_values, key_bytes: int = 256,
                 metadata_bytes_per_block: int = 8, aggregate: bool = True,
                 absolute_margins: dict | None = None, wave: int = 1):
    """The reference's replay sweep over one trace (replay.py:476-627): a
    pandas DataFrame of per-transition rows, or their aggregate."""

    import pandas as pd

    frame = pd.DataFrame(replay_trace_rows(
        trace, k_values=k_values, block_sizes=block_sizes, gamma_sigma_values=gamma_sigma_values,
        key_bytes=key_bytes, metadata_bytes_per_block=metadata_bytes_per_block, absolute_margins=absolute_margins,
        wave=wave))
    return aggregate_rows(frame) if aggregate else frame


def aggregate_rows(frame):
    """Group per-transition rows and summarise them (replay.py:592-627)."""

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
# Statistics tables of consecutive rows (reference replay.py:403-474).
# ---------------------------------------------------------------------------
def _moments(x: torch.Tensor, y: torch.Tensor, abs_delta: torch.Tensor | None = None) -> list[float]:
    """dsa_pair_moments: [mean x, mean y, Sxx, Syy, Sxy, mean d, Sdd]."""

    out = torch.empty(7, device=x.device, dtype=torch.float64)
    code = _lib.DTYPE_F64 if x.dtype == torch.float64 else _lib.DTYPE_F32
    _lib.call("dsa_pair_moments", _lib.ptr(x), _lib.ptr(y), code, x.numel(), _lib.ptr(out), _lib.ptr(abs_delta),
              _lib.stream_of(x))
    return out.tolist()


def _pearson(m: list[float], n: int) -> float:
    """Pearson's r from the moments (reference metrics.py:40-47: NaN for
    fewer than two values or a constant row)."""

    sxx, syy, sxy = m[2], m[3], m[4]
    if n < 2 or sxx == 0.0 or syy == 0.0:
        return math.nan
    return float(min(1.0, max(-1.0, sxy / math.sqrt(sxx * syy))))


def _sorted_desc(row: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The row sorted by (value desc, index asc) with its keys, on the GPU."""

    from .metrics import _exact_topk

    order, values = _exact_topk(row.reshape(1, -1), row.numel(), sorted=True, return_values=True)
    return order[0], values[0]


def _ranks(row: torch.Tensor) -> torch.Tensor:
    order, values = _sorted_desc(row)
    ranks = torch.empty(row.numel(), device=row.device, dtype=torch.float64)
    code = _lib.DTYPE_F64 if values.dtype == torch.float64 else _lib.DTYPE_F32
    _lib.call("dsa_average_ranks", _lib.ptr(values), code, _lib.ptr(order), row.numel(), _lib.ptr(ranks),
              _lib.stream_of(row))
    return ranks


def _percentiles(sorted_desc: torch.Tensor, qs) -> list[float]:
    """numpy's linear percentiles of a row sorted descending, with numpy's
    arithmetic: the quantile q / 100, the virtual index (n - 1) q, its
    fraction and the two-sided lerp are all in the row's own precision
    (float32 rows give float32 percentiles).  Only the two neighbours of each
    virtual index are read back."""

    dt = np.float32 if sorted_desc.dtype == torch.float32 else np.float64
    n = sorted_desc.numel()
    plan = []
    for q in qs:
        qf = dt(q) / dt(100)
        virtual = dt(n - 1) * qf
        if virtual >= n - 1:
            lo = hi = n - 1
        elif virtual < 0:
            lo = hi = 0
        else:
            lo = int(np.floor(virtual))
            hi = lo + 1
        plan.append((lo, hi, dt(virtual - dt(np.floor(virtual)))))
    picks = torch.tensor([n - 1 - i for lo, hi, _ in plan for i in (lo, hi)], device=sorted_desc.device)
    vals = sorted_desc.index_select(0, picks).cpu().numpy().astype(dt)
    out = []
    for j, (_, _, t) in enumerate(plan):
        a, b = vals[2 * j], vals[2 * j + 1]
        diff = dt(b - a)
        out.append(float(dt(b - diff * (dt(1) - t)) if t >= 0.5 else dt(a + diff * t)))
    return out


def temporal_stats(trace: ScoreTrace, k_values):
    """The reference's ``temporal_stats`` (replay.py:403-428) on the GPU: per
    transition and k, the Pearson and Spearman correlations of consecutive
    rows, the drift's mean, std and 99th percentile of |drift|, and the top-k
    overlap.  Returns a pandas DataFrame with the reference's columns."""

    import pandas as pd

    _lib.load()
    dev = torch.device("cuda", torch.cuda.current_device())
    records = []
    for step in range(1, trace.scores.shape[0]):
        prev_h, cur_h = trace.row(step - 1), trace.row(step)
        n = min(prev_h.size, cur_h.size)
        prev = torch.from_numpy(prev_h[:n]).to(dev)
        cur = torch.from_numpy(cur_h[:n]).to(dev)
        abs_delta = torch.empty(n, device=dev, dtype=torch.float32)
        m = _moments(prev, cur, abs_delta)
        rank_m = _moments(_ranks(prev), _ranks(cur))
        p99 = _percentiles(_sorted_desc(abs_delta)[1], [99])[0]
        base = {
            "step": step, "layer": trace.layer, "workload": trace.workload, "prompt_id": trace.prompt_id,
            "context_length": int(cur_h.size),
            "score_pearson": _pearson(m, n),
            "score_spearman": _pearson(rank_m, n),
            "delta_mean": m[5],
            "delta_std": math.sqrt(m[6] / n),
            "delta_p99_abs": p99,
        }
        for k in k_values:
            if k > n:
                continue
            a = device_topk(prev.reshape(1, -1), k, sorted=False)[0]
            b = device_topk(cur.reshape(1, -1), k, sorted=False)[0]
            hits = torch.zeros(1, device=dev, dtype=torch.int32)
            _lib.call("dsa_index_overlap", _lib.ptr(a), _lib.ptr(b), k, _lib.ptr(hits), _lib.stream_of(a))
            records.append({**base, "k": k, "topk_overlap": int(hits.item()) / k})
    return pd.DataFrame(records)


def block_temporal_stats(trace: ScoreTrace, block_sizes, k_values):
    """The reference's ``block_temporal_stats`` (replay.py:431-474) on the
    GPU: per transition, block size and k, the drift of the block maxima
    (mean, 5th / 50th / 95th percentiles) and the fraction of blocks whose
    maximum stayed below the current k-th largest score for at least 1, 2, 4
    and 8 consecutive steps.  Returns a pandas DataFrame with the reference's
    columns."""

    import pandas as pd

    _lib.load()
    dev = torch.device("cuda", torch.cuda.current_device())
    capacity = int(trace.scores.shape[1])
    streaks: dict[tuple[int, int], torch.Tensor] = {}
    records = []
    for step in range(1, trace.scores.shape[0]):
        prev_h, cur_h = trace.row(step - 1), trace.row(step)
        n = min(prev_h.size, cur_h.size)
        prev = torch.from_numpy(prev_h[:n]).to(dev).reshape(1, -1)
        cur = torch.from_numpy(cur_h[:n]).to(dev).reshape(1, -1)
        kth = {k: device_topk(cur, k, sorted=True, return_values=True)[1][0] for k in k_values if k <= n}
        for bs in block_sizes:
            pm = block_max(prev, bs)[0]
            cm = block_max(cur, bs)[0]
            nb = cm.numel()
            for k in k_values:
                if k > n:
                    continue
                state = streaks.setdefault((bs, k), torch.zeros(-(-capacity // bs), device=dev, dtype=torch.int32))
                delta = torch.empty(nb, device=dev, dtype=torch.float64)
                counts = torch.zeros(4, device=dev, dtype=torch.int32)
                _lib.call("dsa_block_streaks", _lib.ptr(pm), _lib.ptr(cm), nb, kth[k].data_ptr() + 4 * (k - 1),
                          _lib.ptr(state), _lib.ptr(delta), _lib.ptr(counts), _lib.stream_of(cm))
                dm = _moments(delta, delta)
                sorted_delta = _sorted_desc(delta)[1]
                p5, p95 = _percentiles(sorted_delta, [5, 95])
                mid = sorted_delta.index_select(0, torch.tensor(sorted({(nb - 1) // 2, nb // 2}), device=dev))
                median = float(mid.double().mean().item()) if mid.numel() == 2 else float(mid[0].item())
                c = counts.tolist()
                records.append({
                    "step": step, "layer": trace.layer, "workload": trace.workload, "prompt_id": trace.prompt_id,
                    "context_length": int(cur_h.size), "k": k, "block_size": bs,
                    "topk_threshold": float(kth[k][k - 1].item()),
                    "delta_max_mean": dm[0],
                    "delta_max_p5": p5,
                    "delta_max_median": median,
                    "delta_max_p95": p95,
                    "cold_fraction_1": c[0] / nb,
                    "cold_fraction_2": c[1] / nb,
                    "cold_fraction_4": c[2] / nb,
                    "cold_fraction_8": c[3] / nb,
                })
    return pd.DataFrame(records)
