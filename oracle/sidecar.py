"""CPU restatement of the sidecar encoders (reference sidecar.py:10-88).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the HIP
encoder projections and epilogues, never by the product path.

Follows, per op, the rounding torch applies in the tensor's dtype:
  * ``apply_noninterleaved_rope`` (sidecar.py:10-28): inv_freq = theta ^
    (-arange(half) / half) and angle = position * inv_freq in float32; cos and
    sin rounded to the row dtype; first*cos - second*sin and second*cos +
    first*sin with every product and sum rounded to the row dtype (bfloat16
    rounding is emulated on float32 values);
  * ``LayerNorm`` (sidecar.py:58, eps 1e-6): float32 mean, biased variance
    and (x - mean) * rstd * weight + bias, rounded once to the row dtype;
  * ``project``: the bias-free Linear projections (sidecar.py:55-58) in
    float64, rounded once to the Linear's dtype;
  * ``encode_keys`` (sidecar.py:74-76) = RoPE(LayerNorm(projection));
    ``encode_queries`` (sidecar.py:78-88) = RoPE on every head of the
    projection, head weights = projection * (heads * head_dim) ^ -0.5 (fp32).

Pinned in tests/test_oracle_sidecar.py against closed forms: identity at
position 0, the float64 rotation, preserved pair norms, rotation by -p
undoing +p, LayerNorm's zero mean / unit variance, bfloat16 rounding
against torch's own cast, and for ``project`` an identity weight, a
hand-computed product whose sum lands exactly between two bfloat16 values
(ties to even), a non-square weight with distinct rows (a transposed
operand fails it) and torch's own float64 matmul.
"""

from __future__ import annotations

import numpy as np


def round_bf16(x) -> np.ndarray:
    """Nearest-even rounding of float32 values to bfloat16, as float32."""

    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(nan, x, r).astype(np.float32)


def inv_freq(half: int, theta: float) -> np.ndarray:
    """theta ^ (-arange(half) / half) in float32 (sidecar.py:20)."""

    exponent = (-np.arange(half, dtype=np.float32)) / np.float32(half)
    return np.power(np.float32(theta), exponent).astype(np.float32)


def apply_noninterleaved_rope(x, positions, *, theta: float = 10_000.0, bf16: bool = False) -> np.ndarray:
    """RoPE of x [..., d] (sidecar.py:10-28); positions has shape x.shape[:-1]
    or x.shape[:-2] (one position per token, broadcast over heads)."""

    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1]
    if d % 2:
        raise ValueError("RoPE dimension must be even")
    half = d // 2
    pos = np.asarray(positions).astype(np.float32)
    angles = (pos[..., None] * inv_freq(half, theta)).astype(np.float32)
    cos = np.cos(angles).astype(np.float32)
    sin = np.sin(angles).astype(np.float32)
    while cos.ndim < x.ndim:
        cos = cos[..., None, :]
        sin = sin[..., None, :]
    rnd = round_bf16 if bf16 else (lambda v: np.asarray(v, dtype=np.float32))
    cos, sin = rnd(cos), rnd(sin)
    first, second = x[..., :half], x[..., half:]
    out1 = rnd(rnd(first * cos) - rnd(second * sin))
    out2 = rnd(rnd(second * cos) + rnd(first * sin))
    return np.concatenate((out1, out2), axis=-1).astype(np.float32)


def partial_rope(x, positions, rope_dim: int, *, theta: float = 10_000.0, bf16: bool = False) -> np.ndarray:
    """The sidecar's _rope (sidecar.py:67-72): RoPE on the first rope_dim dims."""

    x = np.asarray(x, dtype=np.float32)
    if rope_dim == 0:
        return x.copy()
    head = apply_noninterleaved_rope(x[..., :rope_dim], positions, theta=theta, bf16=bf16)
    return np.concatenate((head, x[..., rope_dim:]), axis=-1)


def layer_norm(x, weight, bias, eps: float = 1e-6, *, bf16: bool = False) -> np.ndarray:
    """LayerNorm over the last dim in float32, rounded once to the row dtype."""

    x = np.asarray(x, dtype=np.float32)
    mean = x.mean(axis=-1, keepdims=True, dtype=np.float32)
    centered = (x - mean).astype(np.float32)
    var = (centered * centered).mean(axis=-1, keepdims=True, dtype=np.float32)
    rstd = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    y = (centered * rstd * np.asarray(weight, np.float32) + np.asarray(bias, np.float32)).astype(np.float32)
    return round_bf16(y) if bf16 else y


def project(hidden, weight, *, bf16: bool = False, scale: float | None = None) -> np.ndarray:
    """A bias-free Linear (sidecar.py:55-58, the projections of :74-88):
    hidden [..., k] @ weight [features, k].T computed in float64, then
    rounded as torch stores the Linear's output: to float32, and then to
    bfloat16 for a bf16 Linear (this double rounding differs from a single
    one by a bfloat16 ulp only when the float32 value is a tie; the kernels
    are held to one ulp), times ``scale`` as one float32 product when given
    (weights_proj's head-weight scale)."""

    exact = np.asarray(hidden, dtype=np.float64) @ np.asarray(weight, dtype=np.float64).T
    out = exact.astype(np.float32)
    if bf16:
        return round_bf16(out)
    if scale is not None:
        out = (out * np.float32(scale)).astype(np.float32)
    return out


def encode_keys_epilogue(proj, ln_weight, ln_bias, positions, rope_dim: int, *, eps: float = 1e-6,
                         theta: float = 10_000.0, bf16: bool = False) -> np.ndarray:
    """encode_keys after wk: RoPE(LayerNorm(proj)) (sidecar.py:74-76)."""

    keys = layer_norm(proj, ln_weight, ln_bias, eps, bf16=bf16)
    return partial_rope(keys, positions, rope_dim, theta=theta, bf16=bf16)


def encode_queries_epilogue(proj, proj_weights, positions, rope_dim: int, *, theta: float = 10_000.0,
                            bf16: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """encode_queries after wq / weights_proj (sidecar.py:78-88): proj
    [..., heads, dim], proj_weights [..., heads] fp32."""

    proj = np.asarray(proj, dtype=np.float32)
    heads, dim = proj.shape[-2:]
    queries = partial_rope(proj, positions, rope_dim, theta=theta, bf16=bf16)
    scale = np.float32((heads * dim) ** -0.5)
    weights = (np.asarray(proj_weights, dtype=np.float32) * scale).astype(np.float32)
    return queries, weights
