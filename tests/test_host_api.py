"""Host-side logic of the dsa_amd API (no device needed): head-id validation,
QK accounting, and the input contract errors of the GPU entry points."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsa_amd import metrics, progressive_kernel as P, sidecar, verifier_scoring


def test_split_head_ids_returns_complement() -> None:
    selected, remaining = P.split_head_ids(torch.tensor([0, 2, 4, 6, 8, 10, 12, 63]))
    assert selected.numel() == 8 and remaining.numel() == 56
    assert set(selected.tolist()).isdisjoint(remaining.tolist())
    assert sorted(selected.tolist() + remaining.tolist()) == list(range(64))


@pytest.mark.parametrize("values", [[0, 1], [0, 1, 2, 3, 4, 5, 6, 64], [0, 1, 2, 3, 4, 5, 6, 6]])
def test_split_head_ids_rejects_invalid(values) -> None:
    with pytest.raises(ValueError):
        P.split_head_ids(torch.tensor(values))


def test_dynamic_head_ids_host_weights_is_stable_for_ties() -> None:
    weights = torch.zeros(64)
    weights[20] = -4
    weights[3] = 4
    result = P.dynamic_head_ids(weights)
    assert result[:2].tolist() == [3, 20] and result[2:].tolist() == [0, 1, 2, 4, 5, 6]


def test_progressive_qk_reduction() -> None:
    assert P.progressive_qk_reduction(8192, 0, 0) == pytest.approx(0.875)
    assert P.progressive_qk_reduction(8192, 128, 0) == pytest.approx(0.0)
    work = 2048 * 64 + 6144 * 8 + 1024 * 56
    assert P.progressive_qk_reduction(8192, 32, 16) == pytest.approx(1 - work / (8192 * 64))
    with pytest.raises(ValueError):
        P.progressive_qk_reduction(8192, 129, 0)
    with pytest.raises(ValueError):
        P.progressive_qk_reduction(8192, -1, 0)


def test_gpu_entry_points_reject_host_tensors() -> None:
    q = torch.zeros(64, 128, dtype=torch.bfloat16)
    w = torch.zeros(64)
    k = torch.zeros(65, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensors"):
        P.full_scores_hip(q, w, k)
    with pytest.raises(ValueError, match="GPU tensors"):
        P.progressive_scores_triton(q, w, k, torch.arange(8), torch.zeros(2, dtype=torch.bool), 0.0)
    with pytest.raises(ValueError):
        sidecar.score_encoded(q[None, None], w[None, None], k[None])
    with pytest.raises(ValueError):
        metrics.topk(torch.zeros(10), 3)
    with pytest.raises(ValueError):
        verifier_scoring.score_head_sparse(q[None], w[None], k, [0])


def test_stable_topk_validates_like_the_reference() -> None:
    with pytest.raises(ValueError, match="expected a vector"):
        metrics.stable_topk(np.ones((2, 2)), 1)
    with pytest.raises(ValueError, match="invalid"):
        metrics.stable_topk(np.ones(3), 4)


def test_recall_helpers() -> None:
    assert metrics.topk_recall(np.array([1, 2]), np.array([2, 3])) == 0.5
    assert metrics.normalized_recall_lift(0.5, 2, 4) == 0.0
    assert metrics.topk_recall(torch.tensor([5]), torch.tensor([5])) == 1.0


def test_reference_names_are_aliases() -> None:
    assert P.full_scores_triton is P.full_scores_hip
    assert P.progressive_scores_triton is P.progressive_scores_hip
    assert P.two_pass_scores_triton is P.two_pass_scores_hip
    assert math.ceil(65 / 64) == 2


def test_stable_topk_rejects_nan_and_unsupported_inputs() -> None:
    # NaN has no place in the reference's partition-based order.
    with pytest.raises(ValueError, match="NaN"):
        metrics.stable_topk(np.array([1.0, np.nan, 0.5]), 1)
    with pytest.raises(ValueError, match="dtype"):
        metrics.stable_topk(np.array(["a", "b"]), 1)


def test_workspace_cache_grows_geometrically() -> None:
    # A decode loop whose context grows by one key per step must not keep a
    # workspace per length: the shared buffer at least doubles when it grows,
    # so 64 steps from L=16384 reallocate O(log L) times at most.
    from dsa_amd import _lib

    cpu = torch.device("cpu")
    allocations = 0
    last = None
    for step in range(64):
        need = 1000 * (16384 + step)
        ws = _lib.workspace("test_growth", cpu, 0, need, zeroed=True)
        assert ws.numel() >= need
        if ws is not last:
            allocations += 1
            assert not ws.any()
            last = ws
    assert allocations <= 2
    big = _lib.workspace("test_growth", cpu, 0, 10**6, zeroed=False)
    assert big is last  # a smaller request reuses the buffer


def test_projection_width_mismatch_raises_on_the_host() -> None:
    # The HIP projection kernels take no weight width, so a hidden state whose
    # width differs from the weight's must never reach them: the host raises.
    module = sidecar.LightningIndexerSidecar(hidden_size=64, heads=4, head_dim=32, rope_dim=8).to(torch.bfloat16)
    hidden = torch.zeros(2, 96, dtype=torch.bfloat16)
    with torch.no_grad(), pytest.raises(ValueError, match="does not match"):
        module._project(hidden, module.wq.weight)
    with torch.no_grad():
        assert module._project_pair(hidden, module.wq.weight, module.weights_proj.weight.float()) is None


def test_zeroed_workspaces_are_kept_per_row_count() -> None:
    # A zeroed workspace's zero region (per-row histograms at offset 0) grows
    # with the row count over space that calls with fewer rows use for other
    # data, so a buffer is never shared between row counts.
    from dsa_amd import _lib

    cpu = torch.device("cpu")
    small = _lib.workspace("test_rows", cpu, 0, 1000, zeroed=True, rows=3)
    small.fill_(7)  # what a 3-row call leaves past its histograms
    large = _lib.workspace("test_rows", cpu, 0, 1000, zeroed=True, rows=16)
    assert large is not small and not large.any()
    assert _lib.workspace("test_rows", cpu, 0, 1000, zeroed=True, rows=3) is small


@pytest.mark.parametrize("values,dtype", [
    ([2**63, 2**63 + 1], np.uint64),  # would round into a tie broken by index (the reference returns [1])
    ([-(2**63), 5], np.int64),        # abs() of -2^63 overflows, so the extremes are compared directly
    ([2**53 + 1, 1], np.int64),
    ([-(2**53) - 1, 1], np.int64),
])
def test_exact_order_rejects_integers_beyond_float64(values, dtype) -> None:
    with pytest.raises(ValueError, match="2\\^53"):
        metrics._exact_dtype(torch.from_numpy(np.array(values, dtype=dtype)))


def test_exact_order_keeps_integers_within_float64() -> None:
    for values, dtype in (([2**53, 7], np.uint64), ([-(2**53), 7], np.int64), ([3, 1], np.uint32)):
        got = metrics._exact_dtype(torch.from_numpy(np.array(values, dtype=dtype)))
        assert got.dtype == torch.float64 and [int(v) for v in got.tolist()] == values


def test_replay_percentiles_follow_numpy() -> None:
    # The statistics tables read two neighbours of each virtual index from a
    # descending GPU sort and interpolate on the host with numpy's arithmetic
    # in the row's precision (reference replay.py:420, 461-463 np.percentile);
    # checked here on CPU tensors against numpy itself.
    import numpy as np
    import torch

    from dsa_amd import replay

    rng = np.random.default_rng(0)
    for trial in range(400):
        n = int(rng.integers(1, 3000))
        dt = np.float32 if trial % 2 else np.float64
        x = (rng.standard_normal(n) * rng.uniform(0.1, 10)).astype(dt)
        if trial % 5 == 0:
            x = np.round(x)
        desc = torch.from_numpy(np.sort(x)[::-1].copy())
        got = replay._percentiles(desc, [1, 5, 50, 95, 99, 100])
        assert got == [float(np.percentile(x, q)) for q in (1, 5, 50, 95, 99, 100)]
