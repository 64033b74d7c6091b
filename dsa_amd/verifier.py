"""Two-path verifier as a live decode step on the GPU.

The reference replays its verifier offline (reference verifier.py:173-432
``verifier_step`` / ``replay_verifier_trace``) over recorded dense and
verifier score rows.  :func:`verifier_step` is the runtime-legal step: the
own-trajectory temporal scan of :func:`dsa_amd.approx.approx_step`, then a
cheap current-query score of every key the scan left unscored (the head path
over selected heads, or the dim path over a per-key sketch of a few rotated,
optionally quantized dims), a rescue of the best cold blocks, full scores for
their keys and the exact top-k of the union.  ``state`` is advanced in place
like the reference's ``apply_rescue_to_state`` (verifier.py:103-170).

:class:`VerifierConfig` keeps the reference's fields, defaults and checks
(verifier.py:15-43).  :func:`verifier_metrics` computes the reference's
per-step metrics dict (verifier.py:227-375) from a step's outputs and the
dense scores of the same step (an offline analysis: a live step has no dense
baseline).
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Any

import numpy as np
import torch

from . import _lib
from .approx import RISK_MODELS, ApproxPolicy, ApproxState, _order_code
from .metrics import topk as device_topk
from .progressive_kernel import HEAD_DIM, HEADS
from .temporal import BLOCK_SIZES, _workspace

PATHS = {"head": 0, "dim": 1}


@dataclass(frozen=True)
class VerifierConfig:
    """Runtime-legal current-query candidate generator (reference
    verifier.py:15-43; same fields, defaults and checks).  ``score_ratio`` is
    the verifier's MAC cost per cold key relative to one full 64x128 score."""

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


@dataclass
class VerifierStep:
    """Outcome of one verifier step for ``B`` sequences."""

    topk: torch.Tensor  # int64 [B, k]: the exact top-k of the candidate union, ascending index
    scores: torch.Tensor  # fp32 [B, L]: full scores of the union, -inf elsewhere
    verifier_scores: torch.Tensor  # fp32 [B, L]: verifier scores of cold keys, -inf elsewhere
    block_scores: torch.Tensor  # fp32 [B, blocks]: largest cold verifier score, -inf without cold keys
    cold_count: torch.Tensor  # uint8 [B, blocks]: cold keys per block
    evaluated_blocks: torch.Tensor  # bool [B, blocks]: blocks the temporal scan refreshed
    rescued_blocks: torch.Tensor  # bool [B, blocks]
    ranking: torch.Tensor  # int32 [B, blocks]: cold blocks in rescue order, then -1
    qk_scored: torch.Tensor  # int32 [B]: keys the temporal scan scored
    counts: torch.Tensor  # int32 [B, 4]: cold keys, cold blocks, rescued blocks, rescued cold keys


def verifier_step(
    state: ApproxState,
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    *,
    policy: ApproxPolicy,
    config: VerifierConfig,
    step: int,
    head_ids: torch.Tensor | None = None,
    query_sketch: torch.Tensor | None = None,
    key_sketch: torch.Tensor | None = None,
    sketch_scale: float | None = None,
    promotion_threshold: float | None = None,
    wave: int = 1,
    fallback_value: float | None = None,
    gamma: torch.Tensor | None = None,
    key_scales: torch.Tensor | None = None,
) -> VerifierStep:
    """One live verifier step; advances ``state`` in place.

    Inputs as :func:`dsa_amd.approx.approx_step`.  The head path takes
    ``head_ids`` (``[width]`` shared, or ``[B, width]`` per sequence, e.g.
    :func:`dsa_amd.verifier_scoring.dynamic_head_indices`).  The dim path takes
    ``query_sketch`` (bf16 ``[B, 64, width]``, see :func:`sketch_queries`) and
    ``key_sketch`` (``[B, capacity, width]``: int8 codes with ``sketch_scale``,
    or bf16 values, see :func:`sketch_keys`).  ``promotion_threshold``
    switches from the rescue budget to a fixed threshold (verifier.py:207-216).
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
    if block_size != config.block_size:
        raise ValueError("the state and the verifier config disagree on block_size")
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
    spec = _lib.VerifierSpecC(
        path=PATHS[config.path], width=int(config.width), promotion=0 if promotion_threshold is None else 1,
        sketch_codes=0, rescue_fraction=float(config.rescue_fraction),
        promotion_threshold=0.0 if promotion_threshold is None else float(promotion_threshold), sketch_scale=0.0,
    )
    ids = None
    id_stride = 0
    sketch_stride = 0
    if config.path == "head":
        if head_ids is None:
            raise ValueError("the head path needs head_ids")
        ids = torch.as_tensor(head_ids, device=device).to(torch.int32).contiguous()
        if ids.shape[-1] != config.width or ids.ndim not in (1, 2) or (ids.ndim == 2 and ids.shape[0] != batch):
            raise ValueError(f"head_ids must be [{config.width}] or [batch,{config.width}]")
        if not 0 < config.width <= HEADS:
            raise ValueError("between 1 and 64 head ids are supported")
        # no range check here (it would sync the host every step): the kernel
        # gives an id outside [0, 64) a zero row and weight
        id_stride = 0 if ids.ndim == 1 else ids.stride(0)
    else:
        if query_sketch is None or key_sketch is None:
            raise ValueError("the dim path needs query_sketch and key_sketch")
        if queries.dtype != torch.bfloat16:
            raise ValueError("the dim path takes BF16 queries")
        if config.width % 8 or not 8 <= config.width <= HEAD_DIM:
            raise ValueError("the sketch width must be a multiple of 8 in [8, 128]")
        if query_sketch.shape != (batch, HEADS, config.width) or query_sketch.dtype != torch.bfloat16:
            raise ValueError(f"query_sketch must be bf16 [batch,64,{config.width}]")
        if key_sketch.ndim != 3 or key_sketch.shape[0] != batch or key_sketch.shape[2] != config.width:
            raise ValueError(f"key_sketch must be [batch,capacity,{config.width}]")
        if key_sketch.shape[1] < length:
            raise ValueError("key_sketch holds fewer keys than the context")
        if key_sketch.dtype == torch.int8:
            if sketch_scale is None or not sketch_scale > 0:
                raise ValueError("int8 sketch codes need a positive sketch_scale")
            spec.sketch_codes = 1
            spec.sketch_scale = float(sketch_scale)
        elif key_sketch.dtype != torch.bfloat16:
            raise ValueError("key_sketch must hold int8 codes or bf16 values")
        query_sketch = query_sketch.contiguous()
        key_sketch = key_sketch.contiguous()
        sketch_stride = key_sketch.shape[1]
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
    pol = _lib.ApproxPolicyC(
        gamma=float(policy.gamma), age_slope=float(policy.age_slope), ema_alpha=float(policy.ema_alpha),
        volatility_lambda=float(policy.volatility_lambda), risk_model=RISK_MODELS[policy.risk_model], order=order,
        buckets=buckets, cold_streak=int(policy.cold_streak), age_cap=-1 if policy.age_cap is None else int(policy.age_cap),
        recent_window=int(policy.recent_window), full_refresh=int(full_refresh), history=0,
    )
    queries = queries.contiguous()
    weights = weights.to(torch.float32).contiguous()
    stream = _lib.stream_of(keys)
    f32 = dict(device=device, dtype=torch.float32)
    out = VerifierStep(
        topk=torch.empty((batch, k), device=device, dtype=torch.int64),
        scores=torch.empty((batch, length), **f32),
        verifier_scores=torch.empty((batch, length), **f32),
        block_scores=torch.empty((batch, blocks), **f32),
        cold_count=torch.empty((batch, blocks), device=device, dtype=torch.uint8),
        evaluated_blocks=torch.empty((batch, blocks), device=device, dtype=torch.uint8),
        rescued_blocks=torch.empty((batch, blocks), device=device, dtype=torch.uint8),
        ranking=torch.empty((batch, blocks), device=device, dtype=torch.int32),
        qk_scored=torch.empty(batch, device=device, dtype=torch.int32),
        counts=torch.empty((batch, 4), device=device, dtype=torch.int32),
    )
    ws = _workspace(device, stream, batch, length, k, block_size)
    _lib.call(
        "dsa_verifier_step", _lib.ptr(queries), _lib.ptr(weights), _lib.ptr(keys), key_stride, _lib.ptr(key_scales),
        ctypes.addressof(pol), _lib.ptr(gamma), previous_length, _lib.ptr(state.topk), _lib.ptr(state.last_max),
        _lib.ptr(state.ema), _lib.ptr(state.volatility), _lib.ptr(state.age), _lib.ptr(state.cold_streak), cap_blocks,
        ctypes.addressof(spec), _lib.ptr(ids), id_stride, _lib.ptr(query_sketch), _lib.ptr(key_sketch), sketch_stride,
        _lib.ptr(out.scores), _lib.ptr(out.verifier_scores), _lib.ptr(out.block_scores), _lib.ptr(out.cold_count),
        _lib.ptr(out.evaluated_blocks), _lib.ptr(out.rescued_blocks), _lib.ptr(out.ranking), _lib.ptr(out.topk),
        _lib.ptr(out.qk_scored), _lib.ptr(out.counts), batch, length, k, block_size, wave, _lib.dtype_code(keys.dtype),
        _lib.ptr(ws), ws.numel(), stream,
    )
    out.evaluated_blocks = out.evaluated_blocks.view(torch.bool)
    out.rescued_blocks = out.rescued_blocks.view(torch.bool)
    state.topk = out.topk
    state.length = length
    return out


# ---------------------------------------------------------------------------
# Dim-path sketches.
# ---------------------------------------------------------------------------
def _dims_tensor(dims, width_limit: int, device) -> torch.Tensor:
    d = torch.as_tensor(dims, device=device).to(torch.int32).reshape(-1).contiguous()
    if d.numel() == 0:
        raise ValueError("at least one dimension is needed")
    if bool(((d < 0) | (d >= width_limit)).any()):
        raise ValueError("dimension index out of range")
    return d


def dim_sketch(x: torch.Tensor, dims, *, rotation: str = "hadamard", bits: int | None = None,
               scale: float | None = None, codes: bool = False) -> torch.Tensor:
    """Rotate (normalized Hadamard over the last axis), keep ``dims`` and
    optionally quantize rows of ``x [..., D]`` (D a power of two <= 128) on the
    GPU: values ``[..., width]`` in x's dtype, or int8 codes (``codes=True``).
    With ``bits`` and no ``scale`` the tensor scale max|v| / limit of the
    rotated, selected values is used (one host sync, as the reference's
    ``.cpu()``)."""

    if not x.is_cuda:
        raise ValueError("HIP kernels require GPU tensors")
    if rotation not in ("none", "hadamard"):
        raise ValueError("rotation must be 'none' or 'hadamard'")
    if bits is not None and bits not in (2, 4, 8):
        raise ValueError("bits must be one of 2, 4, 8")
    if codes and bits is None:
        raise ValueError("codes need bits")
    dim = x.shape[-1]
    if dim <= 0 or dim & (dim - 1) or dim > 128:
        raise ValueError("Hadamard dimension must be a positive power of two <= 128")
    dtype = _lib.dtype_code(x.dtype)
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError("sketch rows must be fp32, fp16 or bf16")
    d = _dims_tensor(dims, dim, x.device)
    width = d.numel()
    x = x.contiguous()
    rows = x.numel() // dim
    stream = _lib.stream_of(x)
    if bits is not None and scale is None:
        values = torch.empty((*x.shape[:-1], width), device=x.device, dtype=x.dtype)
        _lib.call("dsa_dim_sketch", _lib.ptr(x), rows, dim, dtype, _lib.ptr(d), width, int(rotation == "hadamard"), 0,
                  0.0, _lib.ptr(values), 0, stream)
        scale = _tensor_scale(values, bits)
        return fake_quantize(values, bits, scale, codes=codes)
    out = torch.empty((*x.shape[:-1], width), device=x.device, dtype=torch.int8 if codes else x.dtype)
    if bits is not None:
        scale = max(float(scale), 1e-12)
    _lib.call("dsa_dim_sketch", _lib.ptr(x), rows, dim, dtype, _lib.ptr(d), width, int(rotation == "hadamard"),
              0 if bits is None else bits, 0.0 if bits is None else scale, _lib.ptr(out), int(codes), stream)
    return out


def _tensor_scale(values: torch.Tensor, bits: int) -> float:
    """max|v| / limit in float64, at least 1e-12 (verifier_scoring.py:37-39)."""

    limit = 2 ** (bits - 1) - 1
    peak = torch.empty(1, device=values.device, dtype=torch.float32)
    if values.numel():
        _lib.call("dsa_abs_max", _lib.ptr(values), values.numel(), _lib.dtype_code(values.dtype), _lib.ptr(peak),
                  _lib.stream_of(values))
        top = float(peak.item())
    else:
        top = 0.0
    return max(top / max(limit, 1), 1e-12)


def fake_quantize(values: torch.Tensor, bits: int, scale: float, *, codes: bool = False) -> torch.Tensor:
    """Symmetric fake quantization with a fixed scale: values in the input
    dtype, or int8 codes."""

    values = values.contiguous()
    out = torch.empty_like(values, dtype=torch.int8) if codes else torch.empty_like(values)
    _lib.call("dsa_fake_quantize", _lib.ptr(values), values.numel(), _lib.dtype_code(values.dtype), bits,
              float(scale), None if codes else _lib.ptr(out), _lib.ptr(out) if codes else None, _lib.stream_of(values))
    return out


def sketch_keys(keys: torch.Tensor, dims, *, rotation: str = "hadamard", bits: int | None = None,
                scale: float | None = None) -> torch.Tensor:
    """Key sketch for the dim path: int8 codes ``[..., width]`` when ``bits``
    is given (``scale`` is then required: a key cache needs a fixed,
    calibrated scale), else bf16 values."""

    if keys.dtype != torch.bfloat16:
        raise ValueError("the dim path takes BF16 keys")
    if bits is not None and scale is None:
        raise ValueError("quantized key sketches need a fixed scale")
    return dim_sketch(keys, dims, rotation=rotation, bits=bits, scale=scale, codes=bits is not None)


def sketch_queries(queries: torch.Tensor, dims, *, rotation: str = "hadamard", bits: int | None = None,
                   scale: float | None = None) -> torch.Tensor:
    """Query sketch for the dim path: bf16 values ``[..., 64, width]``
    (fake-quantized when ``bits`` is given; tensor scale when ``scale`` is
    None)."""

    if queries.dtype != torch.bfloat16:
        raise ValueError("the dim path takes BF16 queries")
    return dim_sketch(queries, dims, rotation=rotation, bits=bits, scale=scale, codes=False)


# ---------------------------------------------------------------------------
# Offline metrics (host arithmetic over one step's outputs).
# ---------------------------------------------------------------------------
def _keys_of_blocks(blocks: np.ndarray, length: int, block_size: int) -> np.ndarray:
    if blocks.size == 0:
        return np.zeros(0, dtype=np.int64)
    keys = (blocks[:, None] * block_size + np.arange(block_size)[None, :]).ravel()
    return keys[keys < length]


def verifier_metrics(
    result: VerifierStep,
    dense_scores: torch.Tensor,
    *,
    config: VerifierConfig,
    policy: ApproxPolicy,
    step: int,
    row: int = 0,
    promotion_threshold: float | None = None,
    tail_critical_blocks=None,
) -> dict[str, Any]:
    """The reference's metrics dict (verifier.py:227-375) for sequence ``row``
    of a step, given that step's dense scores ``[B, L]`` (GPU)."""

    k = result.topk.shape[1]
    dense = dense_scores[row].to(torch.float32)
    length = dense.numel()
    baseline = device_topk(dense.reshape(1, -1), k, sorted=True)[0].cpu().numpy()
    scores = dense.cpu().numpy()
    approximate = result.topk[row].cpu().numpy()
    # rank order (larger score, then lower index), so sums run in the reference's order
    approximate = approximate[np.lexsort((approximate, -scores[approximate]))]
    exact_ids = np.flatnonzero(np.isfinite(result.scores[row].cpu().numpy()))
    cold_mask = np.isfinite(result.verifier_scores[row].cpu().numpy())
    counts = result.counts[row].cpu().numpy()
    ranking = result.ranking[row].cpu().numpy()
    ranking = ranking[ranking >= 0].astype(np.int64)
    rescued = np.flatnonzero(result.rescued_blocks[row].cpu().numpy()).astype(np.int64)
    bs = config.block_size
    n_cold_blocks = int(counts[1])
    temporal_exact = int(result.qk_scored[row].item())
    rescue_new = int(exact_ids.size - temporal_exact)
    cold_tokens = int(counts[0])

    base_mask = np.zeros(length, dtype=bool)
    base_mask[baseline] = True
    exact_mask = np.zeros(length, dtype=bool)
    exact_mask[exact_ids] = True
    newly_active = baseline[cold_mask[baseline]]
    newly_blocks = np.unique(newly_active // bs)
    rescued_positive = np.intersect1d(rescued, newly_blocks)
    tail = np.asarray([] if tail_critical_blocks is None else tail_critical_blocks, dtype=np.int64)
    rescued_tail = np.intersect1d(rescued, tail)

    # average precision of the rescue ranking for newly active blocks
    if newly_blocks.size:
        hits = np.flatnonzero(np.isin(ranking, newly_blocks)) + 1
        ap = 0.0
        for j, rank in enumerate(hits.tolist(), start=1):
            ap += j / rank
        ap = float(ap / newly_blocks.size)
    else:
        ap = 1.0

    def keep(count: int) -> float:
        count = min(count, baseline.size)
        return 1.0 if count == 0 else float(np.isin(baseline[:count], approximate).sum() / count)

    shift = float(np.max(scores[baseline]))
    mass = float(np.exp(scores[approximate].astype(np.float64) - shift).sum()
                 / max(np.exp(scores[baseline].astype(np.float64) - shift).sum(), 1e-300))

    key_bytes = config.full_key_bytes_per_token
    nb = (length + bs - 1) // bs
    metadata_bytes = nb * config.metadata_bytes_per_block
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
    physical = {}
    for pb in (32, 64, 128):
        base_phys = ((length + pb - 1) // pb) * pb * key_bytes
        if config.path == "head":
            reread_blocks = 0
            if not config.retain_candidate_keys and rescued.size:
                reread_blocks = np.unique(_keys_of_blocks(rescued, length, bs) // pb).size
            phys = base_phys + reread_blocks * pb * key_bytes + metadata_bytes
        else:
            phys = (np.unique(exact_ids // pb).size * pb * key_bytes
                    + np.unique(np.flatnonzero(cold_mask) // pb).size * pb * config.sketch_bytes_per_token
                    + metadata_bytes)
        physical[pb] = float(1.0 - phys / base_phys)
    full_equivalent = temporal_exact + rescue_new + cold_tokens * config.score_ratio
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
        "promotion_fraction_of_cold": float(rescued.size / max(1, n_cold_blocks)),
        "temporal_exact_tokens": temporal_exact,
        "cold_tokens_scanned": cold_tokens,
        "cold_blocks_scanned": n_cold_blocks,
        "rescue_blocks": int(rescued.size),
        "rescue_exact_tokens": rescue_new,
        "candidate_union_tokens": int(exact_ids.size),
        "duplicate_exact_tokens": 0,
        "qk_full_equivalent": float(full_equivalent),
        "net_qk_reduction": float(1.0 - full_equivalent / float(length)),
        "exact_match": bool(np.array_equal(np.sort(approximate), np.sort(baseline))),
        "recall": float(base_mask[approximate].sum() / k),
        "top128_recall": keep(128),
        "top256_recall": keep(256),
        "top512_recall": keep(512),
        "top1024_recall": keep(1024),
        "top2048_recall": keep(2048),
        "index_mass_ratio": mass,
        "newly_active_tokens": int(newly_active.size),
        "newly_active_token_recall": float(exact_mask[newly_active].mean()) if newly_active.size else 1.0,
        "newly_active_blocks": int(newly_blocks.size),
        "newly_active_block_recall": float(rescued_positive.size / newly_blocks.size) if newly_blocks.size else 1.0,
        "detector_ap": ap,
        "rescue_precision": float(rescued_positive.size / rescued.size) if rescued.size else 1.0,
        "tail_critical_blocks": int(tail.size),
        "tail_critical_block_recall": float(rescued_tail.size / tail.size) if tail.size else 1.0,
        "temporal_key_bytes": float(temporal_key_bytes),
        "verifier_key_bytes": float(verifier_key_bytes),
        "sketch_bytes": float(sketch_bytes),
        "rescue_reread_key_bytes": float(reread),
        "metadata_bytes": int(metadata_bytes),
        "total_key_bytes": float(total_key_bytes),
        "ideal_key_byte_reduction": float(1.0 - total_key_bytes / (length * key_bytes)),
        "physical_key_byte_reduction": physical[64],
        "physical_b32_key_byte_reduction": physical[32],
        "physical_b64_key_byte_reduction": physical[64],
        "physical_b128_key_byte_reduction": physical[128],
    }


# ---------------------------------------------------------------------------
# Replay over recorded score rows (the reference's offline driver).
# ---------------------------------------------------------------------------
def verifier_replay_step(
    state: ApproxState,
    current_scores: torch.Tensor,
    verifier_scores: torch.Tensor,
    *,
    policy: ApproxPolicy,
    config: VerifierConfig,
    step: int,
    promotion_threshold: float | None = None,
    wave: int = 1,
) -> VerifierStep:
    """One verifier step over recorded rows (reference verifier.py:173-392 as
    ``replay_verifier_trace`` drives it): the dense scores ``[B, L]`` and the
    verifier scores ``[B, L]`` (only cold keys are read) come from a trace
    instead of from keys.  Advances ``state`` in place like
    :func:`verifier_step`."""

    _lib.load()
    if current_scores.ndim != 2 or verifier_scores.shape != current_scores.shape:
        raise ValueError("expected score rows [batch, L] and verifier rows of the same shape")
    if not (current_scores.is_cuda and verifier_scores.is_cuda):
        raise ValueError("HIP kernels require GPU tensors")
    batch, length = current_scores.shape
    block_size = state.block_size
    if block_size != config.block_size:
        raise ValueError("the state and the verifier config disagree on block_size")
    if block_size not in BLOCK_SIZES:
        raise ValueError(f"block_size must be one of {BLOCK_SIZES}")
    if state.topk.shape[0] != batch:
        raise ValueError("state and rows disagree on the batch")
    if policy.risk_model not in RISK_MODELS:
        raise ValueError(f"unknown risk model: {policy.risk_model}")
    order, buckets = _order_code(policy.order)
    previous_length = state.length
    if length < previous_length:
        raise ValueError("rows are shorter than the state's context")
    blocks = math.ceil(length / block_size)
    cap_blocks = state.last_max.shape[1]
    if blocks > cap_blocks:
        raise ValueError(f"context of {length} keys exceeds the state's capacity of {cap_blocks} blocks")
    k = state.topk.shape[1]
    wave = wave if policy.dynamic_threshold else 0
    if policy.dynamic_threshold and wave < 1:
        raise ValueError("a dynamic policy needs wave >= 1")
    device = current_scores.device
    spec = _lib.VerifierSpecC(
        path=PATHS[config.path], width=int(config.width), promotion=0 if promotion_threshold is None else 1,
        sketch_codes=0, rescue_fraction=float(config.rescue_fraction),
        promotion_threshold=0.0 if promotion_threshold is None else float(promotion_threshold), sketch_scale=0.0,
    )
    full_refresh = bool(policy.name == "full" or (policy.refresh_interval and step % policy.refresh_interval == 0))
    pol = _lib.ApproxPolicyC(
        gamma=float(policy.gamma), age_slope=float(policy.age_slope), ema_alpha=float(policy.ema_alpha),
        volatility_lambda=float(policy.volatility_lambda), risk_model=RISK_MODELS[policy.risk_model], order=order,
        buckets=buckets, cold_streak=int(policy.cold_streak), age_cap=-1 if policy.age_cap is None else int(policy.age_cap),
        recent_window=int(policy.recent_window), full_refresh=int(full_refresh), history=0,
    )
    cur = current_scores.to(torch.float32).contiguous()
    ver = verifier_scores.to(torch.float32).contiguous()
    f32 = dict(device=device, dtype=torch.float32)
    out = VerifierStep(
        topk=torch.empty((batch, k), device=device, dtype=torch.int64),
        scores=torch.empty((batch, length), **f32),
        verifier_scores=torch.empty((batch, length), **f32),
        block_scores=torch.empty((batch, blocks), **f32),
        cold_count=torch.empty((batch, blocks), device=device, dtype=torch.uint8),
        evaluated_blocks=torch.empty((batch, blocks), device=device, dtype=torch.uint8),
        rescued_blocks=torch.empty((batch, blocks), device=device, dtype=torch.uint8),
        ranking=torch.empty((batch, blocks), device=device, dtype=torch.int32),
        qk_scored=torch.empty(batch, device=device, dtype=torch.int32),
        counts=torch.empty((batch, 4), device=device, dtype=torch.int32),
    )
    stream = _lib.stream_of(cur)
    ws = _workspace(device, stream, batch, length, k, block_size)
    _lib.call(
        "dsa_verifier_replay_step", _lib.ptr(cur), length, _lib.ptr(ver), length, ctypes.addressof(pol), None,
        previous_length, _lib.ptr(state.topk), _lib.ptr(state.last_max), _lib.ptr(state.ema),
        _lib.ptr(state.volatility), _lib.ptr(state.age), _lib.ptr(state.cold_streak), cap_blocks,
        ctypes.addressof(spec), _lib.ptr(out.scores), _lib.ptr(out.verifier_scores), _lib.ptr(out.block_scores),
        _lib.ptr(out.cold_count), _lib.ptr(out.evaluated_blocks), _lib.ptr(out.rescued_blocks), _lib.ptr(out.ranking),
        _lib.ptr(out.topk), _lib.ptr(out.qk_scored), _lib.ptr(out.counts), batch, length, k, block_size, wave,
        _lib.ptr(ws), ws.numel(), stream,
    )
    out.evaluated_blocks = out.evaluated_blocks.view(torch.bool)
    out.rescued_blocks = out.rescued_blocks.view(torch.bool)
    state.topk = out.topk
    state.length = length
    return out


def replay_verifier_trace(
    trace,
    verifier_scores,
    *,
    policy: ApproxPolicy,
    config: VerifierConfig,
    k: int = 2048,
    max_transitions: int | None = None,
    tail_labels: dict | None = None,
    detail_callback=None,
    promotion_threshold=None,
    wave: int = 1,
):
    """Replay one trace with recorded or lazily generated verifier scores
    (reference verifier.py:395-432): every step on the GPU, and a pandas
    DataFrame of the reference's per-step metrics.  ``verifier_scores`` is an
    array ``[steps, >= L_t]`` or a callable ``(step, length) -> [length]``;
    ``promotion_threshold`` a float, None or a callable of the same form."""

    import pandas as pd

    from .approx import initialize_state

    device = torch.device("cuda", torch.cuda.current_device())
    lengths = np.asarray(trace.lengths, dtype=np.int64)
    row0 = torch.from_numpy(trace.row(0)).to(device).reshape(1, -1)
    state = initialize_state(row0, k=k, block_size=config.block_size, capacity=int(lengths.max()))
    stop = trace.scores.shape[0] if max_transitions is None else min(trace.scores.shape[0], max_transitions + 1)
    rows = []
    for step in range(1, stop):
        length = int(lengths[step])
        partial = verifier_scores(step, length) if callable(verifier_scores) else verifier_scores[step, :length]
        threshold = promotion_threshold(step, length) if callable(promotion_threshold) else promotion_threshold
        cur = torch.from_numpy(trace.row(step)).to(device).reshape(1, -1)
        ver = torch.as_tensor(np.asarray(partial, dtype=np.float32)[:length]).to(device).reshape(1, -1)
        out = verifier_replay_step(state, cur, ver, policy=policy, config=config, step=step,
                                   promotion_threshold=threshold, wave=wave)
        metrics = verifier_metrics(out, cur, config=config, policy=policy, step=step, promotion_threshold=threshold,
                                   tail_critical_blocks=None if tail_labels is None else tail_labels.get(step))
        metrics.update({"layer": trace.layer, "workload": trace.workload, "prompt_id": trace.prompt_id,
                        "base_context_length": int(lengths[0]) - 1})
        rows.append(metrics)
        if detail_callback is not None:
            detail_callback(step, out)
    return pd.DataFrame(rows)
