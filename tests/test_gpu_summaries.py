"""GPU block summaries against the oracle: per-block score maxima (exact),
per-block key norms and the certified radius (both float64; the radius is
never below the oracle's float64 value)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from dsa_amd import _lib, certified
from oracle import certified as C
from oracle import replay as R

pytestmark = pytest.mark.gpu


# Powers of two up to 128 take the coalesced run kernel; 7 and 200 the per-block one.
@pytest.mark.parametrize("block_size", [1, 16, 32, 64, 128, 7, 200])
def test_block_max_exact(device, block_size) -> None:
    rng = np.random.default_rng(block_size)
    host = rng.normal(size=(3, 1001)).astype(np.float32)
    x = torch.from_numpy(host).to(device)
    blocks = -(-1001 // block_size)
    out = torch.empty(3, blocks, device=device)
    _lib.call("dsa_block_max", x.data_ptr(), 3, 1001, 1001, block_size, out.data_ptr(), _lib.stream_of(x))
    for r in range(3):
        np.testing.assert_array_equal(out[r].cpu().numpy(), R.block_maxima(host[r], block_size).astype(np.float32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_key_norms(device, dtype) -> None:
    rng = np.random.default_rng(2)
    keys = torch.from_numpy(rng.normal(size=(70, 3, 128)).astype(np.float32)).to(dtype)
    out = certified.block_key_norms(keys.to(device), 16)
    assert out.dtype == torch.float64
    got = out.cpu().numpy()
    want = C.block_key_norms(keys.float().numpy(), 16)
    np.testing.assert_allclose(got, want, rtol=1e-14)
    shared = certified.block_key_norms(keys[:, 0].to(device), 8).cpu().numpy()
    np.testing.assert_allclose(shared, C.block_key_norms(keys[:, :1].float().numpy(), 8), rtol=1e-14)


def test_temporal_radius(device) -> None:
    rng = np.random.default_rng(1582)
    q_prev = rng.normal(size=(64, 128))
    q_now = q_prev + 0.05 * rng.normal(size=(64, 128))
    w_prev = rng.normal(size=64)
    w_now = w_prev + 0.05 * rng.normal(size=64)
    norms = np.abs(rng.normal(size=(300, 64)))
    want = C.temporal_score_radius(q_now, q_prev, w_now, w_prev, norms)
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731  (float64, as the reference takes them)
    got = certified.temporal_score_radius(t(q_now), t(q_prev), t(w_now), t(w_prev), t(norms)).cpu().numpy()
    # A certified bound must not round below the float64 value, and may sit
    # above it only by the documented (1 + 2^-36) scaling.
    assert np.all(got >= want)
    assert np.all(got <= want * (1 + 2.0**-34))


def test_temporal_radius_asymmetric_closed_form(device) -> None:
    # One head whose query and weight both change, with ||q_now|| != ||q_prev||
    # and |w_now| != |w_prev|: the reference's form (certified.py:43-47) gives
    # |2 - (-1)| * ||(3,4)|| + |2| * ||(6,8)-(3,4)|| = 3*5 + 2*5 = 25, times the
    # block norm 2.  Swapping q_prev for q_now gives 40, w_now for w_prev 20.
    t = lambda a: torch.tensor(a, dtype=torch.float64, device=device)  # noqa: E731
    got = certified.temporal_score_radius(t([[6.0, 8.0]]), t([[3.0, 4.0]]), t([2.0]), t([-1.0]), t([[2.0], [0.5]]))
    want = np.array([50.0, 12.5])
    assert np.all(got.cpu().numpy() >= want) and np.all(got.cpu().numpy() <= want * (1 + 2.0**-34))
