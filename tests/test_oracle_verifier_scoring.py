"""Pins the verifier score oracle (oracle/verifier_scoring.py).

Closed forms and independent constructions only:
  * the normalized Hadamard transform equals x @ H / sqrt(D) with H from
    Sylvester's construction (scipy) in float32 arithmetic, is its own
    inverse and preserves dot products (the reference's own test,
    tests/test_verifier_scoring.py:13-22);
  * its bfloat16 stages round like torch's bfloat16 add / subtract / scalar
    multiply (checked against torch's own bfloat16 ops);
  * fake quantization: codes within +-limit, values on the code * scale grid,
    the max-magnitude element lands on +-limit, re-quantizing is the
    identity, and torch divides by a Python scalar as float32 division;
  * the dim path over all 128 dims equals the head path over all heads (the
    reference's full-width identity, tests/test_verifier_scoring.py:25-32),
    and both equal the float64 closed form sum_h w_h relu(q_h . k).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from scipy.linalg import hadamard

from oracle import verifier_scoring as S
from oracle.scores import relu_index_score
from oracle.sidecar import round_bf16


@pytest.mark.parametrize("size", [2, 8, 128])
def test_hadamard_matches_sylvester_matrix(size) -> None:
    rng = np.random.default_rng(size)
    x = rng.standard_normal((5, size)).astype(np.float32)
    want = (x.astype(np.float64) @ hadamard(size).astype(np.float64)) / np.sqrt(size)
    got = S.normalized_hadamard(x)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5 * np.sqrt(size))
    np.testing.assert_allclose(S.normalized_hadamard(got), x, rtol=0, atol=1e-5)


def test_hadamard_preserves_dot_products() -> None:
    rng = np.random.default_rng(1582)
    q = rng.standard_normal((3, 4, 8)).astype(np.float32)
    k = rng.standard_normal((7, 8)).astype(np.float32)
    direct = np.einsum("qhd,kd->qhk", q, k)
    rotated = np.einsum("qhd,kd->qhk", S.normalized_hadamard(q), S.normalized_hadamard(k))
    np.testing.assert_allclose(direct, rotated, atol=1e-5)


def test_hadamard_rejects_non_power_of_two() -> None:
    with pytest.raises(ValueError):
        S.normalized_hadamard(np.zeros((2, 6)))


def _torch_hadamard(t: torch.Tensor) -> torch.Tensor:
    # torch's bfloat16 arithmetic as the rounding model, stage by stage
    size = t.shape[-1]
    out = t
    stride = 1
    while stride < size:
        g = out.reshape(*out.shape[:-1], -1, 2 * stride)
        out = torch.cat((g[..., :stride] + g[..., stride:], g[..., :stride] - g[..., stride:]), dim=-1).reshape(t.shape)
        stride *= 2
    return out * (size ** -0.5)


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bf16"), (torch.float16, "f16")])
def test_hadamard_stage_rounding_matches_torch_half_arithmetic(dtype, name) -> None:
    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, 128, generator=g).to(dtype)
    want = _torch_hadamard(x).float().numpy()
    got = S.normalized_hadamard(x.float().numpy(), name)
    np.testing.assert_array_equal(got, want)


def test_fake_quantize_closed_forms() -> None:
    rng = np.random.default_rng(11)
    x = round_bf16(rng.standard_normal(4000).astype(np.float32) * 3)
    for bits in (2, 4, 8):
        limit = 2 ** (bits - 1) - 1
        values, scale, codes = S.fake_symmetric_quantize(x, bits, dtype="bf16")
        assert scale == pytest.approx(float(np.abs(x).max()) / limit, rel=1e-15)
        assert np.abs(codes).max() == limit
        assert codes[np.argmax(np.abs(x))] == np.sign(x[np.argmax(np.abs(x))]) * limit
        np.testing.assert_array_equal(values, round_bf16(codes.astype(np.float32) * np.float32(scale)))
        again, _, codes2 = S.fake_symmetric_quantize(values, bits, scale, dtype="bf16")
        np.testing.assert_array_equal(codes2, codes)
        np.testing.assert_array_equal(again, values)
    with pytest.raises(ValueError):
        S.fake_symmetric_quantize(x, 3)


def test_torch_divides_by_python_scalar_in_float32() -> None:
    x = torch.randn(100000, generator=torch.Generator().manual_seed(2)) * 7
    scale = 0.0123456789123
    np.testing.assert_array_equal((x / scale).numpy(), x.numpy() / np.float32(scale))
    np.testing.assert_array_equal(torch.round(torch.tensor([0.5, 1.5, 2.5, -0.5])).numpy(), np.rint([0.5, 1.5, 2.5, -0.5]))


def test_full_width_dim_path_equals_head_path_and_closed_form() -> None:
    rng = np.random.default_rng(1582)
    q = rng.standard_normal((3, 4, 8)).astype(np.float32)
    k = rng.standard_normal((11, 8)).astype(np.float32)
    w = rng.standard_normal((3, 4)).astype(np.float32)
    dim = S.score_dim_sparse(q, w, k, np.arange(8), dtype="f32")
    head = S.weighted_relu_sum(S.head_dots(q, k), w, "f32")
    np.testing.assert_allclose(dim, head, atol=1e-6)
    closed = np.stack([relu_index_score(q[i], k, w[i]) for i in range(3)])
    np.testing.assert_allclose(dim, closed, rtol=1e-6, atol=1e-6)
    # the Hadamard rotation at full width keeps the score up to rounding
    rotated = S.score_dim_sparse(q, w, k, np.arange(8), rotation="hadamard", dtype="f32", round_dots=False)
    np.testing.assert_allclose(rotated, closed, rtol=1e-5, atol=1e-5)


def test_dim_subset_is_partial_sum_of_the_chosen_dims() -> None:
    rng = np.random.default_rng(3)
    q = round_bf16(rng.standard_normal((2, 64, 128)).astype(np.float32))
    k = round_bf16(rng.standard_normal((50, 128)).astype(np.float32))
    w = rng.standard_normal((2, 64)).astype(np.float32)
    dims = np.array([0, 9, 17, 40, 77, 100, 101, 127])
    got = S.score_dim_sparse(q, w, k, dims, dtype="bf16", round_dots=False)
    want = np.stack([relu_index_score(q[i][:, dims], k[:, dims], w[i]) for i in range(2)])
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_layer_energy_dimensions() -> None:
    q = np.zeros((2, 3, 8), dtype=np.float32)
    k = np.zeros((5, 8), dtype=np.float32)
    q[..., [1, 4, 6]] = 1.0
    k[:, [1, 4, 6]] = [2.0, 3.0, 1.0]
    np.testing.assert_array_equal(S.layer_energy_dimensions(q, k, 2), [1, 4])
    # ties keep the lower dimension
    np.testing.assert_array_equal(S.layer_energy_dimensions(np.ones((1, 1, 4)), np.ones((2, 4)), 2), [0, 1])
