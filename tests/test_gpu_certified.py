"""Certified-bound pruning on the GPU.

``certified.certified_margins`` gives every key block a margin that bounds
the change of each of its keys' scores between two steps (the reference's
radius, certified.py:18-48, for a shared-key cache, plus an allowance for the
kernels' fp32 rounding).  A temporal step pruning with ``prev max + margin``
(``temporal_step(..., block_margins=...)``) must then keep every key of the
dense top-k: its top-k equals the dense step's exactly.  The margins are
checked against the float64 oracle (never below it) and, key by key, against
the actual change of the kernels' scores.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsa_amd import certified, decode, temporal
from oracle import certified as C
from oracle import topk as T

pytestmark = pytest.mark.gpu


def drifting(batch, prev_length, length, rho, seed):
    gen = torch.Generator().manual_seed(seed)
    q_prev = torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)
    q_now = rho * q_prev + math.sqrt(1 - rho * rho) * torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)
    w = torch.randn(batch, 64, generator=gen) / 8
    keys = torch.randn(batch, length, 128, generator=gen)
    hot = torch.rand(batch, length, generator=gen) < 0.01
    keys[hot] *= 4
    return q_prev.to(torch.bfloat16), q_now.to(torch.bfloat16), w, keys.to(torch.bfloat16)


def test_margins_match_oracle(device) -> None:
    q_prev, q_now, w, keys = drifting(2, 1000, 1000, 0.99, seed=1)
    w_now = w + 0.01 * torch.randn(w.shape, generator=torch.Generator().manual_seed(2))
    got = certified.certified_margins(q_now.to(device), q_prev.to(device), w_now.to(device), w.to(device),
                                      keys.to(device), 1000, 64).cpu().numpy()
    for b in range(2):
        want = C.certified_margins(q_now[b].float().numpy(), q_prev[b].float().numpy(), w_now[b].numpy(),
                                   w[b].numpy(), keys[b].float().numpy(), 64)
        assert np.all(got[b] >= want) and np.all(got[b] <= want * (1 + 2.0**-34)), b


@pytest.mark.parametrize("block,method,order,wave,rho,must_prune", [
    (16, "dynamic", "previous_hot", 8, 0.99999, True),
    (64, "static", "address", 0, 0.99999, False),
    (32, "dynamic", "upper_hot", 16, 0.999999, True),
    (64, "dynamic", "previous_hot", 32, 0.95, False),
])
def test_certified_step_keeps_the_dense_topk(device, block, method, order, wave, rho, must_prune) -> None:
    print(f"certified bs={block} {method}/{order} wave={wave} rho={rho}", flush=True)
    batch, prev_length, length, k = 2, 8192, 8195, 256
    q_prev, q_now, w, keys = drifting(batch, prev_length, length, rho, seed=block + wave)
    q_prev, q_now, w, keys = q_prev.to(device), q_now.to(device), w.to(device), keys.to(device)
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys[:, :prev_length].contiguous(), k, return_scores=True)
    dense_topk, dense = decode.indexer_topk(q_now, w, keys, k, return_scores=True)
    margins = certified.certified_margins(q_now, q_prev, w, w, keys, prev_length, block)
    # The margin covers every key's change of the kernels' own scores.
    change = (dense[:, :prev_length] - prev_scores).abs().double()
    blocks = math.ceil(prev_length / block)
    pad = torch.zeros(batch, blocks * block, device=device, dtype=torch.float64)
    pad[:, :prev_length] = change
    assert bool((pad.reshape(batch, blocks, block).amax(dim=2) <= margins).all())
    step = temporal.temporal_step(q_now, w, keys, temporal.block_max(prev_scores, block), prev_length, prev_topk, 0.0,
                                  block_size=block, method=method, scan_order=order, wave=max(wave, 1),
                                  block_margins=margins)
    got = step.topk.cpu().numpy()
    host = dense.cpu().numpy()
    for b in range(batch):
        assert got[b].tolist() == T.topk_index_order(host[b], k).tolist(), b
    assert torch.equal(step.topk, dense_topk)
    pruned = int((~step.evaluated_blocks).sum())
    print(f"  pruned {pruned} of {step.evaluated_blocks.numel()} blocks", flush=True)
    if must_prune:
        assert pruned > 0, "a slow drift leaves blocks below the threshold: the case must prune"


def _fp8(keys: torch.Tensor):
    """Keys quantised as C5's: fp8 e4m3fn with scale = max |k| / 448 per 128 keys."""

    raw = keys.float()
    batch, length, _ = raw.shape
    blocks = math.ceil(length / 128)
    pad = torch.zeros(batch, blocks * 128, 128)
    pad[:, :length] = raw
    scales = pad.reshape(batch, blocks, 128 * 128).abs().amax(dim=2) / 448
    keys8 = (raw / scales.repeat_interleave(128, dim=1)[:, :length, None]).to(torch.float8_e4m3fn)
    return keys8, scales


def test_fp8_margins_match_oracle_and_keep_the_dense_topk(device) -> None:
    # fp8 keys (C5's format): the margins are never below the float64 oracle
    # on the dequantised keys (scale * k8), and a certified static and dynamic
    # step over the fp8 keys keep the dense top-k exactly.
    print("certified fp8 keys", flush=True)
    batch, prev_length, length, k, block = 2, 8192, 8195, 256, 64
    q_prev, q_now, w, keys = drifting(batch, prev_length, length, 0.99999, seed=5)
    keys8, scales = _fp8(keys)
    q_prev, q_now, w = q_prev.to(device), q_now.to(device), w.to(device)
    keys8, scales = keys8.to(device), scales.to(device)
    margins = certified.certified_margins(q_now, q_prev, w, w, keys8, prev_length, block, key_scales=scales)
    # scale * k8 in float64 (exact: a float32 product would round each key value)
    deq = (keys8.double() * scales.double().repeat_interleave(128, dim=1)[:, :length, None]).cpu().numpy()
    got = margins.cpu().numpy()
    for b in range(batch):
        want = C.certified_margins(q_now[b].float().cpu().numpy(), q_prev[b].float().cpu().numpy(), w[b].cpu().numpy(),
                                   w[b].cpu().numpy(), deq[b, :prev_length], block)
        assert np.all(got[b] >= want) and np.all(got[b] <= want * (1 + 2.0**-34)), b
    prev_scales = scales[:, : math.ceil(prev_length / 128)].contiguous()
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys8[:, :prev_length].contiguous(), k,
                                                 key_scales=prev_scales, return_scores=True)
    dense_topk, dense = decode.indexer_topk(q_now, w, keys8, k, key_scales=scales, return_scores=True)
    change = (dense[:, :prev_length] - prev_scores).abs().double()
    blocks = math.ceil(prev_length / block)
    pad = torch.zeros(batch, blocks * block, device=device, dtype=torch.float64)
    pad[:, :prev_length] = change
    assert bool((pad.reshape(batch, blocks, block).amax(dim=2) <= margins).all())
    for method, order, wave in (("static", "address", 1), ("dynamic", "previous_hot", 16)):
        step = temporal.temporal_step(q_now, w, keys8, temporal.block_max(prev_scores, block), prev_length, prev_topk,
                                      0.0, block_size=block, method=method, scan_order=order, wave=wave,
                                      key_scales=scales, block_margins=margins)
        assert torch.equal(step.topk, dense_topk), method
        print(f"  {method}: pruned {int((~step.evaluated_blocks).sum())} of {step.evaluated_blocks.numel()} blocks",
              flush=True)
