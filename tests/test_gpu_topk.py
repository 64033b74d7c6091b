"""GPU top-K is bit-exact against the stable_topk oracle (index sets and
order), including ties at the cut-off, signed zeros, -inf, short rows and
the chunked long-row path."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from dsa_amd import metrics
from oracle import topk as T

pytestmark = pytest.mark.gpu


def rows_for(kind: str, rows: int, length: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    if kind == "normal":
        return rng.normal(size=(rows, length)).astype(np.float32)
    if kind == "ties":
        return rng.integers(-3, 4, size=(rows, length)).astype(np.float32)
    if kind == "zeros":
        x = rng.choice(np.array([-0.0, 0.0, 1.0, -1.0], dtype=np.float32), size=(rows, length))
        return x.astype(np.float32)
    if kind == "neginf":
        x = rng.normal(size=(rows, length)).astype(np.float32)
        x[rng.random(size=x.shape) < 0.7] = -np.inf
        return x
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["normal", "ties", "zeros", "neginf"])
@pytest.mark.parametrize("length,k", [(1, 1), (7, 3), (100, 100), (300, 17), (4096, 256), (5000, 4096), (32768, 2048)])
def test_topk_matches_oracle(device, kind, length, k) -> None:
    print(f"topk kind={kind} L={length} k={k}", flush=True)
    host = rows_for(kind, 3, length, seed=length + k)
    x = torch.from_numpy(host).to(device)
    idx_sorted, val_sorted = metrics.topk(x, k, sorted=True, return_values=True)
    idx_index = metrics.topk(x, k, sorted=False)
    for r in range(3):
        want = T.stable_topk(host[r], k)
        assert idx_sorted[r].cpu().numpy().tolist() == want.tolist()
        np.testing.assert_array_equal(val_sorted[r].cpu().numpy(), host[r][want])
        assert idx_index[r].cpu().numpy().tolist() == np.sort(want).tolist()


@pytest.mark.parametrize("kind", ["normal", "ties", "zeros", "neginf"])
@pytest.mark.parametrize("length,k", [(300, 17), (2048, 256), (4096, 512), (4096, 2048)])
def test_many_short_rows(device, kind, length, k) -> None:
    # Enough rows of at most 4096 entries for the 256-thread workgroups (a
    # sorted k above their 1024-entry candidate buffer takes the 1024-thread
    # kernel); every row checked, values bit for bit, with ragged row lengths
    # on half of them.
    print(f"topk many rows kind={kind} L={length} k={k}", flush=True)
    rows = 1536
    host = rows_for(kind, rows, length, seed=7 * length + k)
    rng = np.random.default_rng(length)
    lengths = np.where(np.arange(rows) % 2 == 0, length, rng.integers(0, length + 1, size=rows)).astype(np.int32)
    x = torch.from_numpy(host).to(device)
    lens = torch.from_numpy(lengths).to(device)
    idx_sorted = metrics.topk(x, k, sorted=True, row_lengths=lens).cpu().numpy()
    idx_index, val_index = metrics.topk(x, k, sorted=False, row_lengths=lens, return_values=True)
    idx_index = idx_index.cpu().numpy()
    val_bits = val_index.cpu().numpy().view(np.uint32)
    for r in range(rows):
        n = int(lengths[r])
        assert idx_sorted[r].tolist() == T.topk_sorted_padded(host[r], k, n).tolist(), r
        want = T.topk_index_order(host[r], k, n)
        assert idx_index[r].tolist() == want.tolist(), r
        chosen = want >= 0
        np.testing.assert_array_equal(val_bits[r][chosen], host[r][want[chosen]].view(np.uint32))
        assert np.all(np.isneginf(val_index[r].cpu().numpy()[~chosen]))


@pytest.mark.parametrize("rows", [2049, 3001, 4096])
def test_ragged_rows_beyond_resident(device, rows) -> None:
    # More ragged rows than the chip holds at once (2048 256-thread
    # workgroups), odd counts included.
    print(f"topk ragged rows={rows}", flush=True)
    length, k = 1024, 64
    host = rows_for("ties", rows, length, seed=rows)
    lengths = np.random.default_rng(rows).integers(0, length + 1, size=rows).astype(np.int32)
    lengths[rows // 2] = length
    x = torch.from_numpy(host).to(device)
    lens = torch.from_numpy(lengths).to(device)
    idx_sorted, val_sorted = metrics.topk(x, k, sorted=True, row_lengths=lens, return_values=True)
    idx_index = metrics.topk(x, k, sorted=False, row_lengths=lens).cpu().numpy()
    idx_sorted, val_sorted = idx_sorted.cpu().numpy(), val_sorted.cpu().numpy()
    for r in range(rows):
        n = int(lengths[r])
        want = T.topk_sorted_padded(host[r], k, n)
        assert idx_sorted[r].tolist() == want.tolist(), r
        chosen = want >= 0
        np.testing.assert_array_equal(val_sorted[r][chosen], host[r][want[chosen]])
        assert idx_index[r].tolist() == T.topk_index_order(host[r], k, n).tolist(), r


@pytest.mark.parametrize("kind", ["normal", "ties", "neginf"])
@pytest.mark.parametrize("rows,length,k", [(1, 16384, 2048), (3, 32768, 2048), (2, 50000, 4096), (1, 262144, 100)])
def test_few_long_rows_distributed(device, kind, rows, length, k) -> None:
    # Index-order top-k of a few long rows takes the distributed select; the
    # workspace it shares with the decode step is left ready for reuse.
    print(f"topk distributed kind={kind} rows={rows} L={length} k={k}", flush=True)
    host = rows_for(kind, rows, length, seed=length + rows)
    x = torch.from_numpy(host).to(device)
    for _ in range(2):
        idx, val = metrics.topk(x, k, sorted=False, return_values=True)
        idx, val = idx.cpu().numpy(), val.cpu().numpy()
        for r in range(rows):
            want = T.topk_index_order(host[r], k)
            assert idx[r].tolist() == want.tolist(), r
            np.testing.assert_array_equal(val[r], host[r][want])


def test_row_lengths_pad_short_rows(device) -> None:
    host = rows_for("ties", 4, 600, seed=3)
    lengths = torch.tensor([600, 10, 0, 257], dtype=torch.int32)
    k = 64
    x = torch.from_numpy(host).to(device)
    idx, val = metrics.topk(x, k, sorted=True, row_lengths=lengths.to(device), return_values=True)
    idx2 = metrics.topk(x, k, sorted=False, row_lengths=lengths.to(device))
    for r in range(4):
        n = int(lengths[r])
        assert idx[r].cpu().tolist() == T.topk_sorted_padded(host[r], k, n).tolist()
        assert idx2[r].cpu().tolist() == T.topk_index_order(host[r], k, n).tolist()
        pad = min(n, k)
        assert torch.isneginf(val[r, pad:]).all()


@pytest.mark.parametrize("length", [40000, 131072])
def test_long_rows_use_chunked_merge(device, length) -> None:
    print(f"topk long L={length}", flush=True)
    host = rows_for("ties", 2, length, seed=length)
    host[1] = np.random.default_rng(1).normal(size=length).astype(np.float32)
    x = torch.from_numpy(host).to(device)
    idx = metrics.topk(x, 2048, sorted=True)
    idx_set = metrics.topk(x, 2048, sorted=False)
    for r in range(2):
        want = T.stable_topk(host[r], 2048)
        assert idx[r].cpu().numpy().tolist() == want.tolist()
        assert idx_set[r].cpu().numpy().tolist() == np.sort(want).tolist()


def test_stable_topk_reference_cases(device) -> None:
    assert metrics.stable_topk(np.array([1.0, 3.0, 3.0, 2.0]), 2).tolist() == [1, 2]
    assert np.array_equal(metrics.stable_topk(np.ones(64, dtype=np.float32), 8), np.arange(8))
    gpu = metrics.stable_topk(torch.tensor([0.5, 2.0, 2.0], device=device), 2)
    assert gpu.is_cuda and gpu.cpu().tolist() == [1, 2]


def _f64_rows(kind: str, rows: int, length: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    if kind == "f64_only":
        # distinct in float64, equal once narrowed to float32
        base = rng.integers(0, 50, size=(rows, length)).astype(np.float64)
        return 1.0 + base * 2.0**-40
    if kind == "ties":
        return rng.integers(-3, 4, size=(rows, length)).astype(np.float64)
    if kind == "zeros_inf":
        x = rng.choice(np.array([-0.0, 0.0, 1e300, -1e300, np.inf, -np.inf, 5e-324]), size=(rows, length))
        return x.astype(np.float64)
    return rng.normal(size=(rows, length)) * 1e6


@pytest.mark.parametrize("kind", ["f64_only", "ties", "zeros_inf", "normal"])
@pytest.mark.parametrize("length,k", [(1, 1), (300, 17), (5000, 5000), (40000, 2048), (70000, 9000)])
def test_float64_rows_exact(device, kind, length, k) -> None:
    # stable_topk over float64 (the reference's replay calls it on float64
    # score vectors): values that float32 would merge stay distinct, and the
    # set and order equal the reference definition computed in float64.
    print(f"topk exact f64 kind={kind} L={length} k={k}", flush=True)
    host = _f64_rows(kind, 2, length, seed=length + k)
    x = torch.from_numpy(host).to(device)
    idx_sorted, val_sorted = metrics.topk(x, k, sorted=True, return_values=True)
    idx_index, val_index = metrics.topk(x, k, sorted=False, return_values=True)
    assert val_sorted.dtype == torch.float64
    for r in range(2):
        want = T.stable_topk(host[r], k)
        assert idx_sorted[r].cpu().numpy().tolist() == want.tolist(), r
        # values are x[idx] bit for bit: -0.0 stays -0.0 (it only orders as +0.0)
        np.testing.assert_array_equal(val_sorted[r].cpu().numpy().view(np.uint64), host[r][want].view(np.uint64))
        assert idx_index[r].cpu().numpy().tolist() == np.sort(want).tolist(), r
        np.testing.assert_array_equal(val_index[r].cpu().numpy().view(np.uint64),
                                      host[r][np.sort(want)].view(np.uint64))
    # the reference's own API: a host float64 vector in, a numpy int64 array out
    got = metrics.stable_topk(host[0], k)
    assert isinstance(got, np.ndarray) and got.tolist() == T.stable_topk(host[0], k).tolist()


@pytest.mark.parametrize("kind", ["normal", "ties"])
@pytest.mark.parametrize("length,k", [(9000, 4097), (50000, 20000), (300000, 100)])
def test_float32_large_k_exact(device, kind, length, k) -> None:
    # k above the radix-select kernels' 4096, or any length: the exact kernel.
    print(f"topk exact f32 kind={kind} L={length} k={k}", flush=True)
    host = rows_for(kind, 2, length, seed=length + 3 * k)
    x = torch.from_numpy(host).to(device)
    idx_sorted = metrics.topk(x, k, sorted=True) if k > 4096 else metrics._exact_topk(
        x, k, sorted=True, return_values=False)[0]
    for r in range(2):
        want = T.stable_topk(host[r], k)
        assert idx_sorted[r].cpu().numpy().tolist() == want.tolist(), r


def test_integer_and_bool_inputs(device) -> None:
    ints = np.array([5, -3, 2**52, 7, 7, -2**52, 0], dtype=np.int64)
    assert metrics.stable_topk(ints, 4).tolist() == T.stable_topk(ints, 4).tolist()
    with pytest.raises(ValueError, match="2\\^53"):
        metrics.stable_topk(torch.tensor([2**60, 1], dtype=torch.int64, device=device), 1)


@pytest.mark.parametrize("kind", ["normal", "ties", "neginf"])
@pytest.mark.parametrize("rows,length,k", [(512, 1000, 100), (300, 4096, 512), (2048, 64, 64)])
def test_candidate_lists_many_rows(device, kind, rows, length, k) -> None:
    # dsa_topk over candidate lists (values + their indices; a negative index
    # drops the slot) for many rows: the one-wave-per-row kernel.  Ties go to
    # the earlier slot; the result lists the chosen indices in slot order.
    import ctypes

    from dsa_amd import _lib

    print(f"topk candidate lists kind={kind} rows={rows} L={length} k={k}", flush=True)
    host = rows_for(kind, rows, length, seed=rows + length)
    rng = np.random.default_rng(k)
    ids = rng.integers(0, 1 << 40, size=(rows, length)).astype(np.int64)
    ids[rng.random(size=ids.shape) < 0.2] = -1
    x = torch.from_numpy(host).to(device)
    ids_d = torch.from_numpy(ids).to(device)
    out_idx = torch.empty(rows, k, dtype=torch.int64, device=device)
    out_val = torch.empty(rows, k, dtype=torch.float32, device=device)
    _lib.load()
    _lib.call("dsa_topk", x.data_ptr(), ids_d.data_ptr(), rows, length, length, None, k, 0, out_idx.data_ptr(),
              out_val.data_ptr(), torch.cuda.current_stream(device).cuda_stream)
    got_idx = out_idx.cpu().numpy()
    got_val = out_val.cpu().numpy()
    for r in range(rows):
        valid = np.flatnonzero(ids[r] >= 0)
        sel = T.topk_index_order(host[r][valid], min(k, valid.size))
        slots = valid[sel]
        want = np.full(k, -1, dtype=np.int64)
        want[: slots.size] = ids[r][slots]
        assert got_idx[r].tolist() == want.tolist(), r
        np.testing.assert_array_equal(got_val[r][: slots.size].view(np.uint32), host[r][slots].view(np.uint32))
        assert np.isneginf(got_val[r][slots.size :]).all()
