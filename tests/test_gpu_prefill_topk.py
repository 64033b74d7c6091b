"""GPU parity of the prefill indexer step with its top-k selected inside the
scoring kernel (dsa_score_queries_topk: score_encoded, reference
sidecar.py:89-107, then stable_topk, metrics.py:9-22, per query row).

The scores must equal dsa_score_queries' bit for bit (same streaming code),
and every row's index set must equal the oracle's stable top-k of those
scores over the row's visible keys, in ascending index order, padded with -1
(oracle.topk.topk_index_order), and the separate GPU select (dsa_topk) on
the same rows.  Cases cover the C4 shape, rows resolved by ranking a few keys
of the cut bin and rows resolved by the radix (all-equal and outlier rows),
a causal offset, no mask, ragged lengths, 13 queries per key set (idle waves),
k = 1 and k above the length, fp16, and the selected values.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsa_amd import metrics, sidecar
from oracle import topk as T

pytestmark = pytest.mark.gpu


def _inputs(batch, queries, length, *, seed, dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(batch, queries, 64, 128, generator=gen) / math.sqrt(128)).to(dtype)
    w = torch.randn(batch, queries, 64, generator=gen) / 8
    keys = (torch.randn(batch, length, 128, generator=gen) / math.sqrt(128)).to(dtype)
    return q, w, keys


def _check(device, q, w, keys, k, *, causal, causal_offset=None, values=True):
    batch, nq, length = q.shape[0], q.shape[1], keys.shape[1]
    qd, wd, kd = q.to(device), w.to(device), keys.to(device)
    scores, idx, val = sidecar.score_encoded_topk(qd, wd, kd, k, causal=causal, causal_offset=causal_offset,
                                                  return_values=True)
    plain = sidecar.score_encoded(qd, wd, kd, causal=causal, causal_offset=causal_offset)
    assert torch.equal(scores.view(torch.int32), plain.view(torch.int32))
    offset = (length - nq if causal_offset is None else causal_offset) if causal else None
    vis = np.array([length if offset is None else min(length, t + offset + 1) for t in range(nq)])
    host, got, got_val = scores.cpu().numpy(), idx.cpu().numpy(), val.cpu().numpy()
    for b in range(batch):
        for t in range(nq):
            want = T.topk_index_order(host[b, t], k, int(vis[t]))
            assert got[b, t].tolist() == want.tolist(), (b, t)
            if values:
                sel = want >= 0
                np.testing.assert_array_equal(got_val[b, t][sel], host[b, t][want[sel]])
                assert np.isneginf(got_val[b, t][~sel]).all()
    # The separate GPU select over the same rows agrees.
    rows = torch.as_tensor(np.tile(vis, batch), dtype=torch.int32, device=device)
    sep = metrics.topk(scores.reshape(batch * nq, length), k, sorted=False, row_lengths=rows) if k <= 4096 else None
    if sep is not None:
        assert torch.equal(sep.reshape(batch, nq, -1)[..., :k], idx)


def test_c4_shape(device) -> None:
    print("prefill top-k: C4 T=L=4096 causal k=512", flush=True)
    q, w, keys = _inputs(1, 4096, 4096, seed=1582)
    _check(device, q, w, keys, 512, causal=True, values=False)


@pytest.mark.parametrize("nq,length,k,causal,offset", [
    (64, 1000, 100, True, 936),     # ragged length, causal
    (13, 777, 64, False, None),     # idle waves, no mask
    (40, 4096, 1, True, 0),         # k = 1, one visible key for the first query
    (16, 300, 1500, False, None),   # k above the length: all keys, then -1
    (24, 4096, 4096, True, 4072),   # k = length
])
def test_shapes(device, nq, length, k, causal, offset) -> None:
    print(f"prefill top-k: nq={nq} L={length} k={k} causal={causal} offset={offset}", flush=True)
    q, w, keys = _inputs(2, nq, length, seed=nq * 7 + length)
    _check(device, q, w, keys, k, causal=causal, causal_offset=offset)


def test_fp16(device) -> None:
    print("prefill top-k: fp16", flush=True)
    q, w, keys = _inputs(1, 32, 2048, seed=5, dtype=torch.float16)
    _check(device, q, w, keys, 256, causal=True)


def test_ties_and_outliers(device) -> None:
    # Rows the linear bins cannot split: every score equal (zero weights, so
    # the cut is the k lowest visible indices), every score -0.0 or a negative
    # value (negative weights, keys of zeros among random ones), and rows with
    # one outlier key that puts every other key into the lowest bin.
    print("prefill top-k: ties, signed zeros and outliers", flush=True)
    q, w, keys = _inputs(3, 32, 2048, seed=11)
    w[0] = 0.0
    w[1] = -w[1].abs()
    keys[1, ::3] = 0.0
    keys[2, 1234] *= 4096.0
    _check(device, q, w, keys, 300, causal=False)
    _check(device, q, w, keys, 300, causal=True, causal_offset=1000)
