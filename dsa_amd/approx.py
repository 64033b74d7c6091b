"""Own-trajectory temporal pruning as a live decode step on the GPU.

The reference replays its runtime-legal policy offline over recorded score
traces (reference approx.py:129-364 ``replay_step``): per-block metadata
(stale block max, EMA, volatility, age, cold streak) is advanced only for
blocks a step refreshed, so skipped blocks never see the current scores.
Here that metadata lives on the device and :func:`approx_step` is a real
decode step: the previous approximate top-k seeds the scan, skipped blocks
load no key bytes, and the library advances the metadata in place.

Names and defaults follow the reference: :class:`ApproxPolicy`
(approx.py:15-39), :func:`initialize_state` (approx.py:112-126).  The
reference's ``history_mode="teacher"`` needs the dense step of every
transition and stays an offline analysis; the ``oracle_current`` order reads
the current scores and is rejected for the same reason.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, replace

import numpy as np
import torch

from . import _lib
from .metrics import topk as device_topk
from .progressive_kernel import HEAD_DIM, HEADS
from .temporal import BLOCK_SIZES, TemporalStep, _workspace

RISK_MODELS = {"last_max": 0, "ema": 1}


@dataclass(frozen=True)
class ApproxPolicy:
    """Runtime-legal temporal policy (reference approx.py:15-39; same fields
    and defaults).  ``gamma`` is an absolute score margin."""

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
    """Device policy state of ``B`` sequences (reference approx.py:42-50).

    The metadata rows hold ``capacity_blocks`` blocks each, of which the first
    ``ceil(length / block_size)`` are live; a decode loop appends keys without
    reallocating them.
    """

    topk: torch.Tensor  # int64 [B, k]: the last approximate top-k (the next seeds)
    last_max: torch.Tensor  # fp32 [B, capacity_blocks]
    ema: torch.Tensor  # fp32 [B, capacity_blocks]
    volatility: torch.Tensor  # fp32 [B, capacity_blocks]
    age: torch.Tensor  # int16 [B, capacity_blocks]
    cold_streak: torch.Tensor  # int16 [B, capacity_blocks]
    length: int
    block_size: int
    baseline_topk: torch.Tensor | None = None  # the dense top-k of the last step (replay over recorded rows)
    seed_order: np.ndarray | None = None  # topk in rank order (larger score, then lower index), host

    @property
    def blocks(self) -> int:
        return math.ceil(self.length / self.block_size)

    def host(self) -> dict:
        """The live part of the state as numpy arrays (row-major [B, blocks])."""

        n = self.blocks
        return {
            "topk": self.topk.cpu().numpy(),
            "last_max": self.last_max[:, :n].cpu().numpy(),
            "ema": self.ema[:, :n].cpu().numpy(),
            "volatility": self.volatility[:, :n].cpu().numpy(),
            "age": self.age[:, :n].cpu().numpy(),
            "cold_streak": self.cold_streak[:, :n].cpu().numpy(),
        }


def _order_code(order: str) -> tuple[int, int]:
    if order == "address":
        return 0, 0
    if order in ("previous_max", "predicted_risk"):
        return 1, 0
    if order.startswith("bucket"):
        try:
            buckets = int(order[len("bucket"):])
        except ValueError:
            raise ValueError(f"unknown block order: {order}") from None
        if buckets < 1:
            raise ValueError(f"unknown block order: {order}")
        return 2, buckets
    if order == "oracle_current":
        raise ValueError("the oracle_current order reads the current scores; it is not a runtime step")
    raise ValueError(f"unknown block order: {order}")


def initialize_state(scores: torch.Tensor, *, k: int, block_size: int, capacity: int | None = None) -> ApproxState:
    """State after a dense step (reference approx.py:112-126) for GPU score
    rows ``[B, L]`` (or ``[L]``): the stable top-k, block maxima as last max
    and EMA, zero volatility and age, cold streak 0 for blocks holding a top-k
    key and 1 elsewhere.  ``capacity`` (keys, default L) sizes the metadata
    rows for the context the decode loop will reach."""

    if not scores.is_cuda:
        raise ValueError("initialize_state expects GPU score rows")
    rows = scores.reshape(1, -1) if scores.ndim == 1 else scores
    if rows.ndim != 2:
        raise ValueError("scores must be [batch, L] or [L]")
    rows = rows.to(torch.float32).contiguous()
    batch, length = rows.shape
    if not 0 < k <= length:
        raise ValueError("K cannot exceed the current trace length")
    if block_size < 1:
        raise ValueError("block_size must be positive")
    capacity = length if capacity is None else int(capacity)
    if capacity < length:
        raise ValueError("capacity must hold the current length")
    cap_blocks = math.ceil(capacity / block_size)
    top = device_topk(rows, k, sorted=False)
    dev = rows.device
    state = ApproxState(
        topk=top,
        last_max=torch.empty((batch, cap_blocks), device=dev, dtype=torch.float32),
        ema=torch.empty((batch, cap_blocks), device=dev, dtype=torch.float32),
        volatility=torch.empty((batch, cap_blocks), device=dev, dtype=torch.float32),
        age=torch.empty((batch, cap_blocks), device=dev, dtype=torch.int16),
        cold_streak=torch.empty((batch, cap_blocks), device=dev, dtype=torch.int16),
        length=length,
        block_size=block_size,
        baseline_topk=device_topk(rows, k, sorted=True),  # rank order: the first seeds of a replay
    )
    _lib.call(
        "dsa_approx_init_state", _lib.ptr(rows), length, _lib.ptr(top), _lib.ptr(state.last_max),
        _lib.ptr(state.ema), _lib.ptr(state.volatility), _lib.ptr(state.age), _lib.ptr(state.cold_streak),
        cap_blocks, batch, length, k, block_size, _lib.stream_of(rows),
    )
    return state


def approx_step(
    state: ApproxState,
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    *,
    policy: ApproxPolicy,
    step: int,
    wave: int = 1,
    fallback_value: float | None = None,
    gamma: torch.Tensor | None = None,
    key_scales: torch.Tensor | None = None,
) -> TemporalStep:
    """One own-trajectory decode step for ``B`` sequences; advances ``state``.

    The live counterpart of the reference's ``replay_step(...,
    history_mode="own")`` (approx.py:129-364): queries ``[B, 64, 128]``,
    weights ``[B, 64]``, keys ``[B, L, 128]`` with ``L >= state.length`` (a
    view of a larger cache is read in place; fp8 keys take ``key_scales`` as
    in :func:`dsa_amd.temporal.temporal_step`).  A dynamic policy refreshes
    its threshold after every ``wave`` blocks of the scan (``wave=1`` is the
    reference's schedule).  ``gamma`` (float64 ``[B]``) overrides
    ``policy.gamma`` per sequence.  Returns the step's scores (-inf where not
    scored), refreshed blocks, keys scored and approximate top-k (ascending
    index order); ``state`` then describes this step.
    """

    _lib.load()
    if queries.ndim != 3 or queries.shape[1:] != (HEADS, HEAD_DIM):
        raise ValueError("queries must be [batch,64,128]")
    batch = queries.shape[0]
    if weights.shape != (batch, HEADS):
        raise ValueError("weights must be [batch,64]")
    if keys.ndim != 3 or keys.shape[0] != batch or keys.shape[2] != HEAD_DIM:
        raise ValueError("keys must be [batch,L,128]")
    if not (queries.is_cuda and weights.is_cuda and keys.is_cuda):
        raise ValueError("HIP kernels require GPU tensors")
    block_size = state.block_size
    if block_size not in BLOCK_SIZES:
        raise ValueError(f"block_size must be one of {BLOCK_SIZES}")
    if state.topk.shape[0] != batch:
        raise ValueError("state and queries disagree on the batch")
    if policy.risk_model not in RISK_MODELS:
        raise ValueError(f"unknown risk model: {policy.risk_model}")
    order, buckets = _order_code(policy.order)
    length = keys.shape[1]
    previous_length = state.length
    if length < previous_length:
        raise ValueError("keys are shorter than the state's context")
    blocks = math.ceil(length / block_size)
    cap_blocks = state.last_max.shape[1]
    if blocks > cap_blocks:
        raise ValueError(f"context of {length} keys exceeds the state's capacity of {cap_blocks} blocks")
    k = state.topk.shape[1]
    if policy.dynamic_threshold:
        if wave < 1:
            raise ValueError("a dynamic policy needs wave >= 1")
    else:
        wave = 0
    if keys.stride(2) != 1 or keys.stride(1) != HEAD_DIM:
        keys = keys.contiguous()
    key_stride = keys.stride(0) // HEAD_DIM
    if keys.dtype == torch.float8_e4m3fn:
        if queries.dtype != torch.bfloat16:
            raise ValueError("fp8 keys are scored against BF16 queries")
        if key_scales is None or key_scales.shape != (batch, math.ceil(key_stride / 128)):
            raise ValueError("fp8 keys need key_scales [batch, ceil(capacity/128)]")
        key_scales = key_scales.to(device=keys.device, dtype=torch.float32).contiguous()
    elif queries.dtype not in (torch.float16, torch.bfloat16) or keys.dtype != queries.dtype:
        raise ValueError("queries and keys must share FP16/BF16 dtype")
    device = keys.device
    if gamma is not None:
        gamma = torch.as_tensor(gamma, dtype=torch.float64, device=device).reshape(-1).contiguous()
        if gamma.numel() != batch:
            raise ValueError("gamma must hold one value per sequence")
    fallback = (
        policy.fallback_threshold is not None and fallback_value is not None and fallback_value > policy.fallback_threshold
    )
    full_refresh = bool(
        policy.name == "full" or (policy.refresh_interval and step % policy.refresh_interval == 0) or fallback
    )
    spec = _lib.ApproxPolicyC(
        gamma=float(policy.gamma),
        age_slope=float(policy.age_slope),
        ema_alpha=float(policy.ema_alpha),
        volatility_lambda=float(policy.volatility_lambda),
        risk_model=RISK_MODELS[policy.risk_model],
        order=order,
        buckets=buckets,
        cold_streak=int(policy.cold_streak),
        age_cap=-1 if policy.age_cap is None else int(policy.age_cap),
        recent_window=int(policy.recent_window),
        full_refresh=int(full_refresh),
        history=0,
    )
    queries = queries.contiguous()
    weights = weights.to(torch.float32).contiguous()
    stream = _lib.stream_of(keys)
    scores = torch.empty((batch, length), device=device, dtype=torch.float32)
    evaluated = torch.empty((batch, blocks), device=device, dtype=torch.uint8)
    topk = torch.empty((batch, k), device=device, dtype=torch.int64)
    qk = torch.empty(batch, device=device, dtype=torch.int32)
    ws = _workspace(device, stream, batch, length, k, block_size)
    _lib.call(
        "dsa_approx_step", _lib.ptr(queries), _lib.ptr(weights), _lib.ptr(keys), key_stride, _lib.ptr(key_scales),
        ctypes.addressof(spec), _lib.ptr(gamma), previous_length, _lib.ptr(state.topk), _lib.ptr(state.last_max),
        _lib.ptr(state.ema), _lib.ptr(state.volatility), _lib.ptr(state.age), _lib.ptr(state.cold_streak),
        cap_blocks, _lib.ptr(scores), _lib.ptr(evaluated), _lib.ptr(topk), _lib.ptr(qk), batch, length, k,
        block_size, wave, _lib.dtype_code(keys.dtype), _lib.ptr(ws), ws.numel(), stream,
    )
    state.topk = topk
    state.length = length
    return TemporalStep(topk, scores, evaluated.view(torch.bool), qk)


HISTORY_MODES = {"own": 0, "teacher": 1}


def _policy_struct(policy: ApproxPolicy, full_refresh: bool, history_mode: str = "own") -> "_lib.ApproxPolicyC":
    order, buckets = (3, 0) if policy.order == "oracle_current" else _order_code(policy.order)
    return _lib.ApproxPolicyC(
        gamma=float(policy.gamma), age_slope=float(policy.age_slope), ema_alpha=float(policy.ema_alpha),
        volatility_lambda=float(policy.volatility_lambda), risk_model=RISK_MODELS[policy.risk_model], order=order,
        buckets=buckets, cold_streak=int(policy.cold_streak), age_cap=-1 if policy.age_cap is None else int(policy.age_cap),
        recent_window=int(policy.recent_window), full_refresh=int(full_refresh), history=HISTORY_MODES[history_mode],
    )


def _rank_order(indices: np.ndarray, scores: np.ndarray) -> np.ndarray:
    """indices ordered by larger score, then lower index."""

    indices = np.asarray(indices, dtype=np.int64)
    return indices[np.lexsort((indices, -scores[indices]))]


def _metadata_bytes_per_block(policy: ApproxPolicy) -> int:
    raw = 6 + (1 if policy.order.startswith("bucket") else 0) + (8 if policy.risk_model == "ema" else 0)
    return int(math.ceil(raw / 4) * 4)


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
):
    """One transition replayed over a recorded score row (reference
    approx.py:129-364): the pruning scan, the top-k of the evaluated keys and
    the state update run in the HIP kernels with the row as the score source;
    returns ``(state, metrics, details)`` with the reference's metrics dict
    and details.  ``state`` (one sequence) is advanced in place.  With
    ``history_mode="own"`` the scan is seeded by the previous step's own top-k
    and only refreshed blocks update the state; with ``"teacher"`` it is
    seeded by the previous dense top-k and every block's state is reset from
    the dense row (approx.py:143-158,270-280).  The ``oracle_current`` order is
    available here (the row is known)."""

    if history_mode not in {"own", "teacher"}:
        raise ValueError("history_mode must be 'own' or 'teacher'")
    teacher = history_mode == "teacher"
    _lib.load()
    if state.topk.shape[0] != 1:
        raise ValueError("replay_step takes a one-sequence state")
    if block_size != state.block_size:
        raise ValueError("block_size differs from the state's")
    device = state.topk.device
    host = np.asarray(current_scores.cpu() if isinstance(current_scores, torch.Tensor) else current_scores,
                      dtype=np.float32)
    length = host.size
    if k > length:
        raise ValueError("K cannot exceed the current trace length")
    previous_length = state.length if previous_length is None else int(previous_length)
    blocks = math.ceil(length / block_size)
    cap_blocks = state.last_max.shape[1]
    if blocks > cap_blocks:
        raise ValueError(f"context of {length} keys exceeds the state's capacity of {cap_blocks} blocks")
    if teacher:  # the previous step's dense top-k, in rank order
        seed_host = (state.baseline_topk if state.baseline_topk is not None else state.topk)[0].cpu().numpy()
    else:
        seed_host = state.seed_order
        if seed_host is None:  # right after initialize_state: its top-k in rank order
            seed_host = (state.baseline_topk[0].cpu().numpy() if state.baseline_topk is not None
                         else state.topk[0].cpu().numpy())
    seed_host = seed_host[seed_host < length].astype(np.int64)
    if seed_host.size != k or np.unique(seed_host).size != k:
        raise RuntimeError(f"previous Top-K seed has {seed_host.size} unique keys, expected {k}")
    fallback = bool(policy.fallback_threshold is not None and fallback_value is not None
                    and fallback_value > policy.fallback_threshold)
    full_refresh = bool(policy.name == "full" or (policy.refresh_interval and step % policy.refresh_interval == 0)
                        or fallback)
    if policy.dynamic_threshold and wave < 1:
        raise ValueError("a dynamic policy needs wave >= 1")
    pol = _policy_struct(policy, full_refresh, history_mode)
    row = torch.from_numpy(host).to(device).reshape(1, -1)
    # The current dense top-k in rank order (baseline); the teacher's state
    # update takes its blocks as the hot ones.
    baseline_dev = device_topk(row, k, sorted=True)
    seeds_dev = torch.from_numpy(seed_host).to(device).reshape(1, -1)
    scores = torch.empty((1, length), device=device, dtype=torch.float32)
    evaluated = torch.empty((1, blocks), device=device, dtype=torch.uint8)
    top = torch.empty((1, k), device=device, dtype=torch.int64)
    qk = torch.empty(1, device=device, dtype=torch.int32)
    stream = _lib.stream_of(row)
    ws = _workspace(device, stream, 1, length, k, block_size)
    from .temporal import block_max

    current_max = block_max(row, block_size) if policy.order == "oracle_current" else None
    _lib.call(
        "dsa_approx_replay_step", _lib.ptr(row), length, _lib.ptr(current_max), ctypes.addressof(pol), None,
        previous_length,
        _lib.ptr(seeds_dev), _lib.ptr(baseline_dev) if teacher else None, _lib.ptr(state.last_max), _lib.ptr(state.ema), _lib.ptr(state.volatility),
        _lib.ptr(state.age), _lib.ptr(state.cold_streak), cap_blocks, _lib.ptr(scores), _lib.ptr(evaluated),
        _lib.ptr(top), _lib.ptr(qk), 1, length, k, block_size, wave if policy.dynamic_threshold else 0, _lib.ptr(ws),
        ws.numel(), stream,
    )
    baseline = baseline_dev[0].cpu().numpy()
    scored = np.flatnonzero(np.isfinite(scores[0].cpu().numpy()))
    approximate = _rank_order(top[0].cpu().numpy(), host)
    refreshed = evaluated[0].cpu().numpy().astype(bool)
    approx_mask = np.zeros(length, dtype=bool)
    approx_mask[approximate] = True
    base_mask = np.zeros(length, dtype=bool)
    base_mask[baseline] = True
    previous_baseline = state.baseline_topk.reshape(-1).cpu().numpy() if state.baseline_topk is not None else baseline
    newly_hot = np.setdiff1d(baseline, previous_baseline)
    newly_missed = int((~approx_mask[newly_hot]).sum()) if newly_hot.size else 0
    missed_rank = np.flatnonzero(~approx_mask[baseline]) + 1
    seed_blocks = np.unique(seed_host // block_size)
    meta_bpb = _metadata_bytes_per_block(policy)
    meta = blocks * meta_bpb

    def keep(count: int) -> float:
        count = min(count, baseline.size)
        return float(np.isin(baseline[:count], approximate).sum() / count)

    shift = float(np.max(host[baseline]))
    mass = float(np.exp(host[approximate].astype(np.float64) - shift).sum()
                 / max(np.exp(host[baseline].astype(np.float64) - shift).sum(), 1e-300))
    metrics = {
        "step": step, "context_length": length, "history_mode": history_mode, "policy": policy.name,
        "gamma": policy.gamma, "k": k, "block_size": block_size, "qk_scored": int(scored.size),
        "qk_reduction": float(1.0 - scored.size / length),
        "exact_match": bool(np.array_equal(np.sort(approximate), np.sort(baseline))),
        "recall": float(base_mask[approximate].sum() / k),
    }
    for count in (128, 256, 512, 1024, 2048):
        metrics[f"top{count}_recall"] = keep(count)
    metrics.update({
        "index_mass_ratio": mass,
        "newly_hot_count": int(newly_hot.size),
        "newly_hot_missed": newly_missed,
        "newly_hot_miss_rate": float(newly_missed / newly_hot.size) if newly_hot.size else 0.0,
        "missed_count": int(missed_rank.size),
        "worst_missed_rank": int(missed_rank.min()) if missed_rank.size else 0,
        "tau_seed": float(np.min(host[seed_host])),
        "tau_final": float(np.min(host[approximate])),
        "full_refresh": full_refresh,
        "fallback": fallback,
        "blocks_refreshed": int(refreshed.sum()),
        "blocks_skipped": int(blocks - refreshed.sum()),
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
    evaluated_keys = np.zeros(length, dtype=bool)
    evaluated_keys[scored] = True
    for entries in (0, 256, 512, 1024, 2048):
        uncached = evaluated_keys.copy()
        uncached[seed_host[: min(entries, seed_host.size)]] = False
        hbm = int(uncached.sum())
        metrics[f"cache{entries}_hbm_keys"] = hbm
        metrics[f"cache{entries}_net_bf16_reduction"] = float(1.0 - (hbm * 256 + meta) / (length * 256))
    details = {
        "approximate": approximate,
        "baseline": baseline,
        "evaluated": scored,
        "seed": seed_host.copy(),
        "refreshed_blocks": np.flatnonzero(refreshed).astype(np.int32),
        "skipped_blocks": np.flatnonzero(~refreshed).astype(np.int32),
        "missed_ranks": missed_rank.astype(np.int32),
    }
    state.topk = torch.from_numpy(approximate).to(device).reshape(1, -1)
    state.seed_order = approximate
    state.baseline_topk = baseline_dev
    state.length = length
    return state, metrics, details
