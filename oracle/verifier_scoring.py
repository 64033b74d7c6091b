"""CPU restatement of the verifier score paths (test oracle).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the HIP
sketch and verifier kernels, never by the product path.

Reference: verifier_scoring.py:9-139, 162-170.
  * ``normalized_hadamard`` (:9-26): log2(D) butterfly stages
    (left + right, left - right over pairs ``stride`` apart), each sum
    rounded to the tensor dtype, then one multiply by D^-0.5 (float32 scalar,
    rounded to the dtype).
  * ``fake_symmetric_quantize`` (:29-41): limit = 2^(bits-1) - 1; scale =
    max|x| / limit in float64 unless given, at least 1e-12; codes =
    clamp(round_half_even(x_f32 / float32(scale)), -limit, limit); values =
    codes * float32(scale) rounded to the dtype.  (torch divides a float32
    tensor by a Python scalar as a float32 division, checked in the tests.)
  * ``score_dim_sparse`` (:95-139): rotate, keep the chosen dimensions,
    fake-quantize, then sum_h w_h relu(q_h . k) over all heads.
  * ``layer_energy_dimensions`` (:162-170): the ``width`` dimensions of
    largest mean(q^2) * mean(k^2), ascending.

The reference's einsum rounds each head's dot product to the input dtype
(bfloat16) before the ReLU; ``score_dim_sparse`` takes ``round_dots`` to
follow that (default) or to keep float32 dots (the HIP kernels' choice).

Pinned in tests/test_oracle_verifier_scoring.py: the Hadamard matrix against
Sylvester's construction in float64, orthonormality (H H = I, dot products
preserved, the reference's own test), per-stage bfloat16 rounding against
torch's bfloat16 arithmetic, quantization closed forms (codes in range,
values on the grid, idempotence), and the reference's full-width identity
(dim path at all dims == head path at all heads).
"""

from __future__ import annotations

import numpy as np

from .sidecar import round_bf16


def _rounder(dtype: str):
    if dtype == "bf16":
        return round_bf16
    if dtype == "f16":
        return lambda v: np.asarray(v, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "f32":
        return lambda v: np.asarray(v, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype}")


def normalized_hadamard(x, dtype: str = "f32") -> np.ndarray:
    """Orthonormal Walsh-Hadamard transform over the last axis, rounded to
    ``dtype`` after every stage like the reference's tensor ops."""

    rnd = _rounder(dtype)
    out = rnd(np.asarray(x, dtype=np.float32))
    size = out.shape[-1]
    if size <= 0 or size & (size - 1):
        raise ValueError("Hadamard dimension must be a positive power of two")
    stride = 1
    while stride < size:
        grouped = out.reshape(*out.shape[:-1], -1, 2 * stride)
        left, right = grouped[..., :stride], grouped[..., stride:]
        out = np.concatenate((rnd(left + right), rnd(left - right)), axis=-1).reshape(out.shape)
        stride *= 2
    return rnd(out * np.float32(size**-0.5))


def quantize_scale(x, bits: int) -> float:
    """Tensor scale max|x| / limit in float64 (verifier_scoring.py:37-38)."""

    limit = 2 ** (bits - 1) - 1
    return float(np.abs(np.asarray(x, dtype=np.float32)).max()) / max(limit, 1)


def fake_symmetric_quantize(x, bits: int, scale: float | None = None, dtype: str = "f32"):
    """(values in dtype as float32, scale, codes int8)."""

    if bits not in {2, 4, 8}:
        raise ValueError("bits must be one of 2, 4, 8")
    limit = 2 ** (bits - 1) - 1
    x = np.asarray(x, dtype=np.float32)
    if scale is None:
        scale = quantize_scale(x, bits)
    scale = max(float(scale), 1e-12)
    s32 = np.float32(scale)
    codes = np.clip(np.rint(x / s32), -limit, limit).astype(np.float32)
    values = _rounder(dtype)(codes * s32)
    return values, scale, codes.astype(np.int8)


def head_dots(q, k) -> np.ndarray:
    """q [Q,H,D] . k [K,D] -> [Q,H,K] in float64."""

    return np.einsum("qhd,kd->qhk", np.asarray(q, np.float64), np.asarray(k, np.float64))


def weighted_relu_sum(dots, weights, round_dots: str | None) -> np.ndarray:
    """sum_h w_h relu(dot) in float64 from [Q,H,K] dots, optionally rounding
    each dot to a dtype first (the reference einsum's output dtype)."""

    d = np.asarray(dots, dtype=np.float64)
    if round_dots is not None:
        d = _rounder(round_dots)(d.astype(np.float32)).astype(np.float64)
    return (np.maximum(d, 0.0) * np.asarray(weights, np.float64)[:, :, None]).sum(axis=1)


def score_dim_sparse(queries, weights, keys, dims, *, rotation: str = "none", bits: int | None = None,
                     query_scale: float | None = None, key_scale: float | None = None, dtype: str = "bf16",
                     round_dots: bool = True) -> np.ndarray:
    """All-head partial-dimension verifier scores [Q, K] (verifier_scoring.py:95-139)."""

    q = np.asarray(queries, dtype=np.float32)
    k = np.asarray(keys, dtype=np.float32)
    if q.ndim != 3 or np.asarray(weights).shape != q.shape[:2] or k.ndim != 2:
        raise ValueError("expected queries [Q,H,D], weights [Q,H], keys [K,D]")
    rnd = _rounder(dtype)
    q, k = rnd(q), rnd(k)
    if rotation == "hadamard":
        q = normalized_hadamard(q, dtype)
        k = normalized_hadamard(k, dtype)
    elif rotation != "none":
        raise ValueError("rotation must be 'none' or 'hadamard'")
    dims = np.asarray(dims, dtype=np.int64)
    qs, ks = q[..., dims], k[:, dims]
    if bits is not None:
        qs, _, _ = fake_symmetric_quantize(qs, bits, query_scale, dtype)
        ks, _, _ = fake_symmetric_quantize(ks, bits, key_scale, dtype)
    return weighted_relu_sum(head_dots(qs, ks), weights, dtype if round_dots else None)


def layer_energy_dimensions(queries, keys, width: int) -> np.ndarray:
    """The ``width`` dims of largest mean(q^2) * mean(k^2), ascending
    (verifier_scoring.py:162-170; float32 means, stable descending order)."""

    q = np.asarray(queries, dtype=np.float32)
    k = np.asarray(keys, dtype=np.float32)
    energy = (q * q).reshape(-1, q.shape[-1]).mean(axis=0, dtype=np.float32) * (k * k).mean(axis=0, dtype=np.float32)
    order = np.argsort(-energy, kind="stable")[:width]
    return np.sort(order).astype(np.int64)
