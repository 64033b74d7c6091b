"""The allocation-free decode step (dsa_score_topk_noalloc) against the
workspace-taking dsa_score_topk, called through the C ABI.

Calls in a row share the GPU's scratch array.  A one-row call of the
candidate-list plan (64 lists of a 16384-key row) writes its lists from
about 19 KiB to 147 KiB into the array, past its 16 KiB histogram, where the
next call, a sixteen-row call of the histogram plan, keeps its 256 KiB of
histograms: that call is only right if the entry point clears them first.
The C2 shape (list plan), a smaller histogram-plan call and a small list-plan
call follow.  Each must equal dsa_score_topk on the same inputs bit for bit
(scores, indices and values), whatever the previous call left in the array.
Shapes beyond the array are rejected with a clear error.
"""

from __future__ import annotations

import math

import pytest
import torch

from dsa_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(batch, length, seed, device):
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16)
    w = torch.randn(batch, 64, generator=gen) / 8
    keys = torch.randn(batch, length, 128, generator=gen)
    hot = torch.rand(batch, length, generator=gen) < 0.01
    keys[hot] *= 4
    return q.to(device), w.to(device), keys.to(torch.bfloat16).to(device)


def _run(name, q, w, keys, k, *extra):
    batch, length = keys.shape[0], keys.shape[1]
    scores = torch.empty(batch, length, device=keys.device)
    idx = torch.full((batch, k), -7, device=keys.device, dtype=torch.int64)
    val = torch.empty(batch, k, device=keys.device)
    args = [_lib.ptr(q), _lib.ptr(w), _lib.ptr(keys), None, _lib.ptr(scores), batch, length, k, _lib.DTYPE_BF16,
            _lib.ptr(idx), _lib.ptr(val), *extra, _lib.stream_of(keys)]
    _lib.call(name, *args)
    return scores, idx, val


@pytest.mark.parametrize("shapes", [[(1, 16384, 2048, 4), (16, 16384, 6000, 5), (16, 32768, 2048, 1),
                                     (2, 16384, 6000, 2), (3, 4099, 256, 3)]])
def test_noalloc_step_matches_workspace_step(device, shapes) -> None:
    for batch, length, k, seed in shapes:
        print(f"noalloc B={batch} L={length} k={k}", flush=True)
        q, w, keys = _inputs(batch, length, seed, device)
        need = int(_lib.query("dsa_score_topk_workspace_bytes", batch, length))
        ws = torch.zeros(need, device=device, dtype=torch.uint8)
        want = _run("dsa_score_topk", q, w, keys, k, _lib.ptr(ws), need)
        got = _run("dsa_score_topk_noalloc", q, w, keys, k)
        torch.cuda.synchronize()
        for a, b, what in zip(got, want, ("scores", "indices", "values")):
            assert torch.equal(a, b), f"B={batch} L={length} k={k}: {what} differ"


def test_noalloc_rejects_shapes_beyond_its_scratch(device) -> None:
    q, w, keys = _inputs(1, 64, 0, device)
    scores = torch.empty(1, 64, device=device)
    idx = torch.empty(1, 8, device=device, dtype=torch.int64)
    # 16 rows x 262144 keys need 32 MiB of workspace: more than the array holds.
    with pytest.raises(RuntimeError, match="scratch"):
        _lib.call("dsa_score_topk_noalloc", _lib.ptr(q), _lib.ptr(w), _lib.ptr(keys), None, _lib.ptr(scores), 16,
                  262144, 8, _lib.DTYPE_BF16, _lib.ptr(idx), None, _lib.stream_of(keys))
