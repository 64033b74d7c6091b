"""Score traces: the reference's on-disk format, collected on the GPU.

``ScoreTrace``, ``save_trace`` and ``load_trace`` keep the reference's
dataclass, checks and ``.npz`` layout (reference trace.py:11-62): ``scores``
``[steps, max_length]`` (row t holds the scores of keys ``[0, lengths[t])``),
``lengths``, and a JSON ``metadata`` string carrying layer, workload and
prompt id.  Files written here load in the reference's tools and vice versa;
``load_trace`` executes nothing from the file (``allow_pickle=False``).

:func:`collect_trace` produces such a trace from a decode trajectory on the
GPU: every step's dense indexer scores by the HIP scoring kernel, stored as
float16 with -inf padding past each row's length.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np
import torch

from . import _lib
from .progressive_kernel import HEAD_DIM, HEADS


@dataclass(frozen=True)
class ScoreTrace:
    """One layer/prompt trace; row t contains scores for keys [0, lengths[t])."""

    scores: np.ndarray
    lengths: np.ndarray
    layer: int
    workload: str
    prompt_id: str
    metadata: dict[str, Any]

    def __post_init__(self) -> None:
        if self.scores.ndim != 2:
            raise ValueError(f"scores must be [steps,max_length], got {self.scores.shape}")
        if self.lengths.shape != (self.scores.shape[0],):
            raise ValueError("lengths must have one entry per step")
        if np.any(self.lengths <= 0) or np.any(self.lengths > self.scores.shape[1]):
            raise ValueError("lengths are outside the score matrix")

    def row(self, step: int) -> np.ndarray:
        return np.asarray(self.scores[step, : self.lengths[step]], dtype=np.float32)


def save_trace(path: str | Path, trace: ScoreTrace) -> None:
    """Write ``trace`` as the reference's compressed ``.npz``."""

    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    metadata = {**trace.metadata, "layer": trace.layer, "workload": trace.workload, "prompt_id": trace.prompt_id}
    np.savez_compressed(path, scores=trace.scores, lengths=trace.lengths,
                        metadata=np.asarray(json.dumps(metadata, sort_keys=True)))


def load_trace(path: str | Path) -> ScoreTrace:
    """Read a trace written by :func:`save_trace` or by the reference."""

    with np.load(Path(path), allow_pickle=False) as data:
        metadata = json.loads(str(data["metadata"].item()))
        return ScoreTrace(
            scores=data["scores"],
            lengths=data["lengths"],
            layer=int(metadata.pop("layer")),
            workload=str(metadata.pop("workload")),
            prompt_id=str(metadata.pop("prompt_id")),
            metadata=metadata,
        )


def collect_trace(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    lengths,
    *,
    layer: int = 0,
    workload: str = "synthetic",
    prompt_id: str = "0",
    metadata: dict[str, Any] | None = None,
    dtype: np.dtype = np.float16,
) -> ScoreTrace:
    """Dense score trace of one sequence's decode trajectory, on the GPU.

    ``queries`` ``[steps, 64, 128]`` and ``weights`` ``[steps, 64]`` (or
    ``[64]``) are the per-step indexer inputs, ``keys`` ``[max_length, 128]``
    the key cache (fp16/bf16), and ``lengths[t]`` the context length at step
    t.  Each step is scored by ``dsa_full_scores`` on its first ``lengths[t]``
    keys; rows are stored in ``dtype`` (float16 by default, as traces are
    kept) with -inf past each row's length.
    """

    _lib.load()
    if not (queries.is_cuda and weights.is_cuda and keys.is_cuda):
        raise ValueError("HIP kernels require GPU tensors")
    if queries.ndim != 3 or queries.shape[1:] != (HEADS, HEAD_DIM):
        raise ValueError("queries must be [steps,64,128]")
    steps = queries.shape[0]
    if weights.shape == (HEADS,):
        weights = weights.expand(steps, HEADS)
    if weights.shape != (steps, HEADS):
        raise ValueError("weights must be [steps,64] or [64]")
    if keys.ndim != 2 or keys.shape[1] != HEAD_DIM:
        raise ValueError("keys must be [max_length,128]")
    if keys.dtype not in (torch.float16, torch.bfloat16) or queries.dtype != keys.dtype:
        raise ValueError("queries and keys must share FP16/BF16 dtype")
    lengths = np.asarray(lengths, dtype=np.int64)
    if lengths.shape != (steps,) or np.any(lengths <= 0) or np.any(lengths > keys.shape[0]):
        raise ValueError("lengths must hold one length in [1, max_length] per step")
    width = int(lengths.max())
    queries = queries.contiguous()
    weights = weights.to(torch.float32).contiguous()
    keys = keys.contiguous()
    rows = torch.full((steps, width), float("-inf"), device=keys.device, dtype=torch.float32)
    stream = _lib.stream_of(keys)
    for t in range(steps):
        n = int(lengths[t])
        out = rows[t]
        _lib.call("dsa_full_scores", _lib.ptr(queries[t]), _lib.ptr(weights[t]), _lib.ptr(keys), None,
                  _lib.ptr(out), 1, n, _lib.dtype_code(keys.dtype), stream)
    scores = rows.cpu().numpy().astype(dtype)
    return ScoreTrace(scores=scores, lengths=lengths, layer=int(layer), workload=str(workload),
                      prompt_id=str(prompt_id), metadata=dict(metadata or {}))
