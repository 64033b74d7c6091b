"""Pins the sidecar encoder oracle (oracle/sidecar.py) against closed forms:
position 0 is the identity, fp32 RoPE matches the float64 rotation, pair
norms survive, rotating by -p undoes +p, LayerNorm gives zero mean and unit
variance, and bfloat16 rounding agrees with torch's own cast."""

from __future__ import annotations

import numpy as np
import torch

from oracle import sidecar as O


def test_round_bf16_matches_torch_cast() -> None:
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.standard_normal(4096).astype(np.float32) * np.float32(10.0) ** rng.integers(-6, 6, 4096),
        np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-9, -1.0 - 2**-8, 0.0, -0.0, np.inf, -np.inf, 3.3895e38],
                 dtype=np.float32),
    ]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.round_bf16(x), want)


def test_rope_identity_at_position_zero() -> None:
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 3, 16)).astype(np.float32)
    out = O.apply_noninterleaved_rope(x, np.zeros(5, dtype=np.int64))
    np.testing.assert_array_equal(out, x)


def test_rope_matches_float64_rotation_and_keeps_pair_norms() -> None:
    rng = np.random.default_rng(5)
    x = rng.standard_normal((7, 64)).astype(np.float32)
    pos = rng.integers(0, 50_000, 7)
    out = O.apply_noninterleaved_rope(x, pos, theta=10_000.0)
    half = 32
    freq = 10_000.0 ** (-np.arange(half) / half)
    ang = pos[:, None].astype(np.float64) * freq
    a, b = x[:, :half].astype(np.float64), x[:, half:].astype(np.float64)
    want = np.concatenate((a * np.cos(ang) - b * np.sin(ang), b * np.cos(ang) + a * np.sin(ang)), axis=1)
    # float32 angles at positions up to 5e4 carry ~4e-3 rad of rounding; the
    # rotation itself is exact otherwise
    np.testing.assert_allclose(out, want, atol=2e-2 * np.abs(x).max())
    small = O.apply_noninterleaved_rope(x, np.arange(7), theta=10_000.0)
    ang = np.arange(7)[:, None].astype(np.float64) * freq
    want = np.concatenate((a * np.cos(ang) - b * np.sin(ang), b * np.cos(ang) + a * np.sin(ang)), axis=1)
    np.testing.assert_allclose(small, want, rtol=0, atol=1e-5)
    n_in = np.hypot(a, b)
    n_out = np.hypot(out[:, :half].astype(np.float64), out[:, half:].astype(np.float64))
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5, atol=1e-6)


def test_rope_by_minus_p_undoes_plus_p() -> None:
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 2, 32)).astype(np.float32)
    pos = np.array([1, 17, 250, 4095])
    back = O.apply_noninterleaved_rope(O.apply_noninterleaved_rope(x, pos), -pos)
    np.testing.assert_allclose(back, x, rtol=0, atol=1e-5)


def test_bf16_rope_is_bf16_and_close_to_float64() -> None:
    rng = np.random.default_rng(7)
    x = O.round_bf16(rng.standard_normal((6, 4, 64)).astype(np.float32))
    pos = np.arange(6) * 11
    out = O.apply_noninterleaved_rope(x, pos, bf16=True)
    np.testing.assert_array_equal(O.round_bf16(out), out)
    ref = O.apply_noninterleaved_rope(x, pos)
    np.testing.assert_allclose(out, ref, rtol=2**-6, atol=2**-6 * np.abs(x).max())


def test_partial_rope_leaves_the_tail() -> None:
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    out = O.partial_rope(x, np.array([5, 6, 7]), 64)
    np.testing.assert_array_equal(out[:, 64:], x[:, 64:])
    np.testing.assert_array_equal(O.partial_rope(x, np.array([5, 6, 7]), 0), x)


def test_layer_norm_closed_form() -> None:
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((10, 128)) * 3 + 1).astype(np.float32)
    y = O.layer_norm(x, np.ones(128), np.zeros(128)).astype(np.float64)
    np.testing.assert_allclose(y.mean(axis=1), 0.0, atol=1e-5)
    np.testing.assert_allclose(y.var(axis=1), 1.0, rtol=1e-4)
    w = rng.standard_normal(128).astype(np.float32)
    b = rng.standard_normal(128).astype(np.float32)
    z = O.layer_norm(x, w, b)
    np.testing.assert_allclose(z, y * w + b, rtol=1e-5, atol=1e-5)


def test_query_weight_scale() -> None:
    _, weights = O.encode_queries_epilogue(np.zeros((2, 64, 128)), np.full((2, 64), 2.0), np.zeros(2), 64)
    np.testing.assert_allclose(weights, 2.0 / np.sqrt(64 * 128), rtol=1e-7)


def test_project_identity_and_rounding() -> None:
    # Identity weight: the projection is the input itself (bf16 values stay).
    x = O.round_bf16(np.random.default_rng(0).standard_normal((5, 8)).astype(np.float32))
    np.testing.assert_array_equal(O.project(x, np.eye(8), bf16=True), x)
    # 1 + 2^-8 lies exactly between the bf16 values 1 and 1 + 2^-7: ties to
    # even gives 1.  1 + 3 * 2^-8 lies between 1 + 2^-7 and 1 + 2^-6: even is
    # 1 + 2^-6.  (Sums of products 1*1 + 2^-8*1 and 1*1 + 3*2^-8*1.)
    h = np.array([[1.0, 2.0**-8], [1.0, 3 * 2.0**-8]], dtype=np.float32)
    w = np.array([[1.0, 1.0]], dtype=np.float32)
    assert O.project(h, w, bf16=True)[:, 0].tolist() == [1.0, 1.0 + 2.0**-6]
    assert O.project(h, w)[:, 0].tolist() == [1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8]


def test_project_orientation_and_scale() -> None:
    # weight [features=3, k=2] with distinct rows: out[t, f] = sum_k h[t, k] w[f, k].
    h = np.array([[1.0, 10.0], [2.0, 20.0]])
    w = np.array([[1.0, 0.0], [0.0, 1.0], [3.0, -1.0]])
    assert O.project(h, w).tolist() == [[1.0, 10.0, -7.0], [2.0, 20.0, -14.0]]
    assert O.project(h, w, scale=0.5).tolist() == [[0.5, 5.0, -3.5], [1.0, 10.0, -7.0]]
    rng = np.random.default_rng(3)
    hb = rng.standard_normal((7, 64))
    wb = rng.standard_normal((16, 64))
    want = (torch.from_numpy(hb) @ torch.from_numpy(wb).T).float().numpy()
    np.testing.assert_allclose(O.project(hb, wb), want, rtol=1e-6, atol=1e-6)
