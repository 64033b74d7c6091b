"""Top-K selection and recall with the reference's metrics API.

Mirrors ``temporal_dsa.metrics`` (reference ``src/temporal_dsa/metrics.py``).
``stable_topk`` keeps the reference's definition (metrics.py:9-22): the k
largest values, ties at the cut-off resolved towards the lower index, returned
sorted by (value desc, index asc).  It runs on the GPU: float32 rows within
the radix-select kernels' limits (k <= 4096) take those, and everything else
(float64 values, integer arrays, any k up to the row length, any length)
takes the exact 64-bit-key kernel (``dsa_topk_exact``).  Host (numpy) inputs
are copied to the current GPU and the result is returned as a numpy int64
array, like the reference.  NaN values are rejected with ValueError (the
reference's partition-based result is not a top-k for them).
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib

MAX_K = 4096
MAX_ROW = 32768
# A few long rows in index order go through the distributed select (every CU
# works on them) rather than one workgroup per row.
DISTRIBUTED_MAX_ROWS = 16
DISTRIBUTED_MIN_LENGTH = 16384  # below, one workgroup per row is as fast (three launches cost more)
DISTRIBUTED_MAX_LENGTH = 524288


def _device() -> torch.device:
    _lib.load()
    if not torch.cuda.is_available():
        raise RuntimeError("stable_topk runs on the GPU; no HIP device is available")
    return torch.device("cuda", torch.cuda.current_device())


def topk(
    scores: torch.Tensor,
    k: int,
    *,
    sorted: bool = True,
    row_lengths: torch.Tensor | None = None,
    return_values: bool = False,
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """Row-wise stable top-k of a GPU fp32 matrix ``[rows, L]`` (or vector).

    ``sorted=True`` orders each row by (value desc, index asc); ``sorted=False``
    returns the same set in ascending index order.  ``row_lengths`` (int32,
    per row) limits the candidates to a row's first entries; rows with fewer
    than k candidates are padded with index -1 and value -inf.
    """

    if not scores.is_cuda:
        raise ValueError("topk expects a GPU tensor; use stable_topk for host arrays")
    squeeze = scores.ndim == 1
    matrix = scores.reshape(1, -1) if squeeze else scores
    if matrix.ndim != 2:
        raise ValueError(f"expected a vector or a matrix, got {tuple(scores.shape)}")
    matrix = _exact_dtype(matrix)
    if matrix.stride(1) != 1:
        matrix = matrix.contiguous()
    rows, length = matrix.shape
    if length == 0:
        raise ValueError("cannot take top-k of an empty row")
    if k <= 0:
        raise ValueError(f"k={k} must be positive")
    if matrix.dtype == torch.float64 or k > MAX_K:
        # float64 rows, or k beyond the radix-select kernels: the exact kernel.
        if row_lengths is not None:
            raise ValueError(f"row_lengths is supported for float32 rows with k <= {MAX_K}")
        if k > length:
            raise ValueError(f"k={k} exceeds the row length {length} (padding needs float32 rows, k <= {MAX_K})")
        indices, values = _exact_topk(matrix, k, sorted=sorted, return_values=return_values)
        if squeeze:
            indices = indices[0]
            values = values[0] if values is not None else None
        return (indices, values) if return_values else indices
    indices = torch.empty((rows, k), device=matrix.device, dtype=torch.int64)
    values = torch.empty((rows, k), device=matrix.device, dtype=torch.float32) if return_values else None
    stream = _lib.stream_of(matrix)
    if (
        not sorted
        and row_lengths is None
        and rows <= DISTRIBUTED_MAX_ROWS
        and DISTRIBUTED_MIN_LENGTH <= length <= DISTRIBUTED_MAX_LENGTH
    ):
        from .decode import _workspace

        matrix = matrix.contiguous()
        if matrix.data_ptr() % 16:
            # A contiguous slice that starts mid-row (x[1:3] with L % 4 != 0)
            # is not 16-byte aligned, as the distributed kernels need.
            matrix = matrix.clone()
        workspace = _workspace(matrix.device, stream, rows, length)
        _lib.call(
            "dsa_topk_distributed", _lib.ptr(matrix), rows, length, k, _lib.ptr(indices), _lib.ptr(values),
            _lib.ptr(workspace), workspace.numel(), stream,
        )
    elif length <= MAX_ROW:
        lengths = None
        if row_lengths is not None:
            lengths = row_lengths.to(device=matrix.device, dtype=torch.int32).contiguous()
            if lengths.numel() != rows:
                raise ValueError("row_lengths needs one entry per row")
        _lib.call(
            "dsa_topk", _lib.ptr(matrix), None, rows, length, matrix.stride(0), _lib.ptr(lengths),
            k, int(sorted), _lib.ptr(indices), _lib.ptr(values), stream,
        )
    else:
        if row_lengths is not None:
            raise ValueError(f"row_lengths is supported for rows up to {MAX_ROW} entries")
        matrix = matrix.contiguous()
        need = int(_lib.query("dsa_topk_long_workspace_bytes", rows, length, k))
        workspace = torch.empty(max(need, 1), device=matrix.device, dtype=torch.uint8)
        _lib.call(
            "dsa_topk_long", _lib.ptr(matrix), rows, length, k, int(sorted), _lib.ptr(indices),
            _lib.ptr(values), _lib.ptr(workspace), need, stream,
        )
    if squeeze:
        indices = indices[0]
        values = values[0] if values is not None else None
    return (indices, values) if return_values else indices


def _exact_dtype(matrix: torch.Tensor) -> torch.Tensor:
    """The dtype the kernels compare in, without changing any value: float32
    for float32/float16/bfloat16 (exact), float64 for float64 and integers
    (integers beyond 2^53 in magnitude cannot be compared exactly and raise)."""

    if matrix.dtype in (torch.float32, torch.float16, torch.bfloat16):
        return matrix.to(torch.float32)
    if matrix.dtype == torch.float64:
        return matrix
    if matrix.dtype == torch.bool or not matrix.dtype.is_floating_point:
        return _integers_as_float64(matrix)
    raise ValueError(f"unsupported dtype {matrix.dtype}")


def _integers_as_float64(matrix: torch.Tensor) -> torch.Tensor:
    """Integer or bool values as float64, which holds every integer up to
    2^53 in magnitude exactly; anything beyond raises ValueError (it would be
    rounded into a tie, e.g. 2^63 and 2^63 + 1).  The check reads the extremes
    without abs(), which overflows at -2^63; uint64 is read through its int64
    bits, since torch has no reductions over it (a value of 2^63 or more has
    its top bit set and reads negative)."""

    limit = 2**53
    if matrix.dtype == torch.uint64:
        bits = matrix.view(torch.int64)
        if bits.numel() and (bool((bits < 0).any()) or int(bits.max()) > limit):
            raise ValueError("integer values beyond 2^53 in magnitude cannot be ordered exactly")
        return bits.to(torch.float64)
    if matrix.dtype == torch.int64 and matrix.numel():
        if int(matrix.max()) > limit or int(matrix.min()) < -limit:
            raise ValueError("integer values beyond 2^53 in magnitude cannot be ordered exactly")
    return matrix.to(torch.float64)


def _exact_topk(matrix: torch.Tensor, k: int, *, sorted: bool, return_values: bool):
    """dsa_topk_exact on a float32 or float64 GPU matrix (unit column stride)."""

    rows, length = matrix.shape
    code = _lib.DTYPE_F64 if matrix.dtype == torch.float64 else _lib.DTYPE_F32
    indices = torch.empty((rows, k), device=matrix.device, dtype=torch.int64)
    values = torch.empty((rows, k), device=matrix.device, dtype=matrix.dtype) if return_values else None
    stream = _lib.stream_of(matrix)
    need = int(_lib.query("dsa_topk_exact_workspace_bytes", rows, k, int(sorted)))
    workspace = _lib.workspace("topk_exact", matrix.device, stream, need, zeroed=False) if need else None
    _lib.call(
        "dsa_topk_exact", _lib.ptr(matrix), code, rows, length, matrix.stride(0), k, int(sorted), _lib.ptr(indices),
        _lib.ptr(values), _lib.ptr(workspace), need, stream,
    )
    return indices, values


def stable_topk(values: np.ndarray | torch.Tensor, k: int) -> np.ndarray | torch.Tensor:
    """Descending top-k indices with the index as deterministic tie-breaker.

    Reference: metrics.py:9-22 (same validation and messages).  A GPU tensor
    yields a GPU int64 tensor; anything else is copied to the GPU and yields a
    numpy int64 array.  Values are compared exactly in their own precision:
    float32 and narrower in float32, float64 and integers with 64-bit keys.
    NaN values raise ValueError.
    """

    on_gpu = isinstance(values, torch.Tensor) and values.is_cuda
    if isinstance(values, torch.Tensor):
        shape = tuple(values.shape)
        size = values.numel()
    else:
        array = np.asarray(values)
        shape = array.shape
        size = array.size
    if len(shape) != 1:
        raise ValueError(f"expected a vector, got {shape}")
    if not 0 < k <= size:
        raise ValueError(f"k={k} is invalid for {size} values")
    if on_gpu:
        if values.dtype.is_floating_point and bool(torch.isnan(values).any()):
            raise ValueError("stable_topk does not order NaN values")
        return topk(values, k, sorted=True)
    host = values.detach().cpu().numpy() if isinstance(values, torch.Tensor) else array
    if host.dtype.kind == "f" and np.isnan(host).any():
        raise ValueError("stable_topk does not order NaN values")
    if host.dtype.kind not in "fiub":
        raise ValueError(f"unsupported dtype {host.dtype}")
    if host.dtype == np.float16:
        host = host.astype(np.float32)
    device = _device()
    return topk(torch.from_numpy(np.ascontiguousarray(host)).to(device), k, sorted=True).cpu().numpy()


def topk_recall(predicted, target) -> float:
    """Recall@K = |predicted ∩ target| / |target| (reference metrics.py:25-30)."""

    predicted = np.asarray(predicted.cpu() if isinstance(predicted, torch.Tensor) else predicted)
    target = np.asarray(target.cpu() if isinstance(target, torch.Tensor) else target)
    if target.size == 0:
        return 1.0
    return float(np.intersect1d(predicted, target, assume_unique=False).size / target.size)


def normalized_recall_lift(recall: float, k: int, length: int) -> float:
    """Recall lift over random selection (reference metrics.py:33-37)."""

    random_recall = min(1.0, k / length)
    if random_recall == 1.0:
        return 1.0
    return float((recall - random_recall) / (1.0 - random_recall))
