"""Temporal pruning of a decode step on the GPU (seeded, bounded block scan).

The reference evaluates temporal pruning offline: ``replay_transition``
(reference replay.py:225-400) replays a score trace through the filter of
replay.py:172-222.  ``temporal_step`` runs the same filter as a real decode
step: the previous step's top-k keys are scored first, every key block whose
bound ``previous block max + gamma`` falls below the running threshold is
skipped without loading its keys, and the top-k is taken over the keys that
were scored.  Methods follow the reference's names:

- ``static``: threshold fixed at the seeds' minimum, address order;
- ``static_hot_first``: the same decisions, visiting the seeds' blocks first;
- ``dynamic``: the threshold is refreshed to the k-th largest evaluated score
  after every ``wave`` blocks of the scan (``wave=1`` is the reference's
  per-block refresh; a GPU processes a wave of blocks per launch).

``gamma`` is an absolute margin (the reference's calibrated margins,
replay.py:562-590): a live step cannot use the current step's score drift.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from .progressive_kernel import HEAD_DIM, HEADS

BLOCK_SIZES = (16, 32, 64, 128)
SCAN_ORDERS = {"address": 0, "previous_hot": 1, "upper_hot": 2}
METHODS = ("static", "static_hot_first", "dynamic")


@dataclass
class TemporalStep:
    """Outcome of one pruned step (per sequence of the batch)."""

    topk: torch.Tensor  # int64 [B, k], ascending index order
    scores: torch.Tensor  # fp32 [B, L], -inf for keys that were not scored
    evaluated_blocks: torch.Tensor  # bool [B, ceil(L / block_size)]
    qk_scored: torch.Tensor  # int32 [B]
    # int32 [B]: workgroups of the fused static launch whose bounded wait for
    # the row's seed minima ran out; they kept every block of their chunk, so
    # a nonzero row holds a superset of the filter's decisions.  Always 0 on
    # the other paths (and None where the step does not report it).
    waits_given_up: torch.Tensor | None = None


def _workspace(device, stream, batch, length, k, block_size) -> torch.Tensor:
    """Workspace shared by the temporal, own-trajectory and verifier steps on
    one stream.  Zero-filled when allocated: the fused static step's exchange
    slots (a fixed region at its start, the same for every shape) must not
    hold a stamp of a later call; the steps clear everything else they use."""

    need = int(_lib.query("dsa_temporal_workspace_bytes", batch, length, k, block_size))
    return _lib.workspace("temporal", device, stream, need, zeroed=True, rows=0)


def keys_loaded(step: TemporalStep, block_size: int) -> torch.Tensor:
    """Key rows the last dynamic step on the current stream loaded, per row
    (int32 [B]): the seeds plus every key of the blocks its rounds scored, a
    superset of ``step.qk_scored`` (the keys the scan evaluates).  Read from
    the step's workspace, so call it before another step runs on the stream.
    No counterpart in the reference, whose replay prices bytes from the keys
    scored (replay.py:369-371)."""

    batch, length = step.scores.shape
    k = step.topk.shape[1]
    device = step.scores.device
    stream = _lib.stream_of(step.scores)
    ws = _workspace(device, stream, batch, length, k, block_size)
    out = torch.empty(batch, device=device, dtype=torch.int32)
    _lib.call("dsa_temporal_keys_loaded", _lib.ptr(ws), batch, length, k, block_size, _lib.ptr(out), stream)
    return out


def _outputs(device, batch: int, length: int, blocks: int, k: int):
    """The step's outputs as views of one allocation (one allocator call per
    step instead of five): scores fp32 [B, L], top-k int64 [B, k], keys
    scored int32 [B], kept-block flags uint8 [B, blocks] and given-up waits
    int32 [B]."""

    def up(n: int) -> int:
        return (n + 255) // 256 * 256

    sizes = (batch * length * 4, batch * k * 8, batch * 4, batch * blocks, batch * 4)
    offsets, total = [], 0
    for size in sizes:
        offsets.append(total)
        total += up(size)
    buf = torch.empty(total, device=device, dtype=torch.uint8)
    scores = buf[offsets[0] : offsets[0] + sizes[0]].view(torch.float32).view(batch, length)
    topk = buf[offsets[1] : offsets[1] + sizes[1]].view(torch.int64).view(batch, k)
    qk = buf[offsets[2] : offsets[2] + sizes[2]].view(torch.int32)
    evaluated = buf[offsets[3] : offsets[3] + sizes[3]].view(batch, blocks)
    gave_up = buf[offsets[4] : offsets[4] + sizes[4]].view(torch.int32)
    return scores, evaluated, topk, qk, gave_up


def temporal_step(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    previous_block_max: torch.Tensor,
    previous_length: int,
    previous_topk: torch.Tensor,
    gamma,
    *,
    block_size: int = 64,
    method: str = "dynamic",
    scan_order: str = "previous_hot",
    wave: int = 32,
    key_scales: torch.Tensor | None = None,
    block_margins: torch.Tensor | None = None,
) -> TemporalStep:
    """One pruned decode step for ``B`` sequences.

    queries ``[B, 64, 128]``, weights ``[B, 64]``, keys ``[B, L, 128]`` (the
    query dtype, or fp8 e4m3fn with ``key_scales`` ``[B, ceil(C/128)]`` for a
    key buffer of capacity C; a view ``cache[:, :L]`` of a ``[B, C, 128]``
    cache is read in place),
    ``previous_block_max`` ``[B, ceil(previous_length / block_size)]``,
    ``previous_topk`` ``[B, k]`` (distinct indices below ``previous_length``),
    ``gamma`` a float or ``[B]`` tensor, or ``block_margins``
    ``[B, ceil(previous_length / block_size)]`` float64 per-block margins used
    instead of it (e.g. :func:`dsa_amd.certified.certified_margins`).
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
    if block_size not in BLOCK_SIZES:
        raise ValueError(f"block_size must be one of {BLOCK_SIZES}")
    if method not in METHODS:
        raise ValueError(f"unknown method: {method}")
    if method == "static":
        scan_order, wave = "address", 0
    elif method == "static_hot_first":
        scan_order, wave = "previous_hot", 0
    elif wave < 1:
        raise ValueError("dynamic pruning needs wave >= 1")
    if scan_order not in SCAN_ORDERS:
        raise ValueError(f"unknown scan order: {scan_order}")
    length = keys.shape[1]
    if not 0 < previous_length <= length:
        raise ValueError("expected previous length <= current length")
    prev_blocks = math.ceil(previous_length / block_size)
    if previous_block_max.shape != (batch, prev_blocks):
        raise ValueError(f"previous_block_max must be [batch,{prev_blocks}]")
    if previous_topk.ndim != 2 or previous_topk.shape[0] != batch:
        raise ValueError("previous_topk must be [batch,k]")
    k = previous_topk.shape[1]
    if not 0 < k <= previous_length:
        raise ValueError("k must fit the previous step so it can seed the scan")
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
    if isinstance(gamma, torch.Tensor):
        gamma_t = gamma.to(device=device, dtype=torch.float32).reshape(-1)
    else:  # a number: filled on the device (a host tensor would be copied with a synchronising transfer)
        gamma_t = torch.full((batch,), float(gamma), dtype=torch.float32, device=device)
    if gamma_t.numel() == 1:
        gamma_t = gamma_t.expand(batch)
    if gamma_t.numel() != batch:
        raise ValueError("gamma must be a float or one value per sequence")
    queries = queries.contiguous()
    weights = weights.to(torch.float32).contiguous()
    prev_max = previous_block_max.to(device=device, dtype=torch.float32).contiguous()
    seeds = previous_topk.to(device=device, dtype=torch.int64).contiguous()
    gamma_t = gamma_t.contiguous()
    margins = None
    if block_margins is not None:
        if tuple(block_margins.shape) != (batch, prev_blocks):
            raise ValueError(f"block_margins must be [batch,{prev_blocks}]")
        margins = block_margins.to(device=device, dtype=torch.float64).contiguous()
    stream = _lib.stream_of(keys)
    blocks = math.ceil(length / block_size)
    scores, evaluated, topk, qk, gave_up = _outputs(device, batch, length, blocks, k)
    ws = _workspace(device, stream, batch, length, k, block_size)
    _lib.call(
        "dsa_temporal_step", _lib.ptr(queries), _lib.ptr(weights), _lib.ptr(keys), key_stride, _lib.ptr(key_scales),
        _lib.ptr(prev_max), previous_length, _lib.ptr(seeds), _lib.ptr(gamma_t), _lib.ptr(margins), _lib.ptr(scores),
        _lib.ptr(evaluated), _lib.ptr(topk), _lib.ptr(qk), _lib.ptr(gave_up), batch, length, k, block_size,
        SCAN_ORDERS[scan_order], wave, _lib.dtype_code(keys.dtype), _lib.ptr(ws), ws.numel(), stream,
    )
    return TemporalStep(topk, scores, evaluated.view(torch.bool), qk, gave_up)


def block_max(scores: torch.Tensor, block_size: int) -> torch.Tensor:
    """Per-block maxima ``[B, ceil(L / block_size)]`` of GPU score rows
    (reference replay.py:149-150)."""

    if not scores.is_cuda or scores.ndim != 2:
        raise ValueError("block_max expects GPU score rows [B, L]")
    scores = scores.to(torch.float32).contiguous()
    rows, length = scores.shape
    out = torch.empty((rows, math.ceil(length / block_size)), device=scores.device, dtype=torch.float32)
    _lib.call("dsa_block_max", _lib.ptr(scores), rows, length, length, block_size, _lib.ptr(out), _lib.stream_of(scores))
    return out
