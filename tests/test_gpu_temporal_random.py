"""Randomised parity sweep of the dynamic temporal step (the rounds path)
against the oracle's replay filter (reference replay.py:172-222).

Eighteen configurations drawn from a fixed seed, and eight with rows of 8K to
40K keys and k up to 2048 from another, and three whose refresh groups hold
more than 8192 keys with the running k largest: block sizes 16-128, the live
step's three scan orders (oracle_current needs recorded scores: the replay
tests cover it), refresh waves from one block to a whole-row's worth, margins from
-sigma to +sigma, lengths that do and do not grow, k from 8 to 1000, bf16 and
fp16, keys with and without crowds of equal scores, and the round splits the
library accepts.  Each must keep the oracle's blocks, score its number of
keys, carry the dense scores of the keys it evaluates bit for bit, and return
the stable top-k of those scores."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsa_amd import decode, temporal
from oracle import replay as R
from oracle import topk as T

pytestmark = pytest.mark.gpu


def draw_cases(n: int, seed: int) -> list:
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        block = int(rng.choice([16, 32, 64, 128]))
        order = str(rng.choice(["address", "previous_hot", "upper_hot"]))
        k = int(rng.choice([8, 64, 256, 1000]))
        prev_length = int(rng.integers(k + 1, 7000))
        length = prev_length + int(rng.choice([0, 1, 17]))
        blocks = math.ceil(length / block)
        wave = int(rng.integers(1, max(2, blocks // 2)))
        gamma_sigma = float(rng.choice([-1.0, -0.25, 0.0, 0.5, 1.0]))
        dtype = str(rng.choice(["bf16", "f16"]))
        distinct = int(rng.choice([0, 0, 3, 40]))
        splits = str(rng.choice(["1", "0.25", "0.5", "0.1,0.3", "0.05,0.15,0.4,0.8"]))
        cases.append((i, block, order, k, prev_length, length, wave, gamma_sigma, dtype, distinct, splits))
    return cases


CASES = draw_cases(18, seed=1582)


def draw_long_cases(n: int, seed: int) -> list:
    """Longer rows (to 40K keys, past the one-workgroup top-k's 32K), k to
    2048, waves of one or two blocks or up to half the row, within the step's
    limits (at most 2048 blocks; k + wave * block_size <= 8192, which only the
    sequential path requires, is left to the three cases below)."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        k = int(rng.choice([256, 1000, 2048]))
        prev_length = int(rng.integers(8192, 40000))
        length = prev_length + int(rng.choice([0, 1, 200]))
        block = int(rng.choice([b for b in (16, 32, 64, 128) if math.ceil(length / b) <= 2048]))
        order = str(rng.choice(["address", "previous_hot", "upper_hot"]))
        blocks = math.ceil(length / block)
        wave = int(rng.choice([1, 2, int(rng.integers(1, max(2, blocks // 2)))]))
        wave = max(1, min(wave, (8192 - k) // block))
        gamma_sigma = float(rng.choice([-1.0, -0.25, 0.0, 0.5, 1.0, 2.0]))
        dtype = str(rng.choice(["bf16", "f16"]))
        distinct = int(rng.choice([0, 0, 40, 500]))
        splits = str(rng.choice(["1", "0.25", "0.1,0.3", "0.05,0.15,0.4,0.8"]))
        cases.append((100 + i, block, order, k, prev_length, length, wave, gamma_sigma, dtype, distinct, splits))
    return cases


CASES += draw_long_cases(8, seed=2026)
# Refresh groups whose keys, with the running k largest, pass the replay's
# 8192 LDS keys (it sorts them in the workspace instead).
CASES += [
    (200, 64, "address", 2048, 30000, 30001, 128, 0.0, "bf16", 0, "0.25"),
    (201, 128, "previous_hot", 4096, 60000, 60017, 64, -0.25, "f16", 0, "0.1,0.3"),
    (202, 32, "upper_hot", 1000, 20000, 20000, 300, 0.5, "bf16", 40, "1"),
]


def transition(batch, prev_length, length, seed, rho=0.95):
    gen = torch.Generator().manual_seed(seed)
    q_prev = torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)
    q_cur = rho * q_prev + math.sqrt(1 - rho * rho) * torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)
    w = torch.randn(batch, 64, generator=gen) / 8
    keys = torch.randn(batch, length, 128, generator=gen)
    for b in range(batch):
        keys[b, torch.randperm(length, generator=gen)[: max(1, length // 100)]] *= 4
    return q_prev, q_cur, w, keys


@pytest.mark.parametrize("case,block,order,k,prev_length,length,wave,gamma_sigma,dtype,distinct,splits", CASES)
def test_dynamic_step_random_configuration(device, monkeypatch, case, block, order, k, prev_length, length, wave,
                                           gamma_sigma, dtype, distinct, splits) -> None:
    print(f"random dynamic case {case}: bs={block} {order} k={k} L={prev_length}->{length} W={wave} "
          f"gs={gamma_sigma} {dtype} distinct={distinct} splits={splits}", flush=True)
    torch_dtype = torch.bfloat16 if dtype == "bf16" else torch.float16
    batch = 2
    q_prev, q_cur, w, keys = transition(batch, prev_length, length, seed=1000 + case)
    if distinct:
        keys = keys[:, torch.arange(length) % distinct]
    q_prev, q_cur, keys = q_prev.to(torch_dtype), q_cur.to(torch_dtype), keys.to(torch_dtype)
    q_prev, q_cur, w, keys = q_prev.to(device), q_cur.to(device), w.to(device), keys.to(device)
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys[:, :prev_length].contiguous(), k, return_scores=True)
    prev_max = temporal.block_max(prev_scores, block)
    dense = decode.indexer_topk(q_cur, w, keys, k, return_scores=True)[1].cpu().numpy()
    gamma = torch.full((batch,), gamma_sigma * float(prev_scores.std()), device=device)
    monkeypatch.setenv("DSA_AMD_TEMPORAL_ROUNDS", splits)
    step = temporal.temporal_step(q_cur, w, keys, prev_max, prev_length, prev_topk, gamma, block_size=block,
                                  method="dynamic", scan_order=order, wave=wave)
    scores, kept, qk, topk = (x.cpu().numpy() for x in (step.scores, step.evaluated_blocks, step.qk_scored, step.topk))
    seeds = prev_topk.cpu().numpy()
    blocks = math.ceil(length / block)
    for b in range(batch):
        previous_max = np.full(blocks, -np.inf)
        previous_max[: prev_max.shape[1]] = prev_max[b].cpu().double().numpy()
        upper = R.upper_bounds(previous_max, float(gamma[b]), prev_length, length, block)
        hot = np.zeros(blocks, dtype=bool)
        hot[seeds[b] // block] = True
        scan = R.block_scan_order(order, upper, R.block_maxima(dense[b], block), hot)
        current = dense[b].astype(np.float64)
        trace = R.run_filter(current, seeds[b], k, block, upper, scan, dynamic=True,
                             fixed_threshold=float(current[seeds[b]].min()), wave=wave)
        np.testing.assert_array_equal(kept[b], trace.kept, err_msg=f"row {b}: kept blocks")
        assert int(qk[b]) == trace.scored, (b, int(qk[b]), trace.scored)
        ev = trace.evaluated
        np.testing.assert_array_equal(scores[b][ev], dense[b][ev])
        assert np.isneginf(scores[b][~ev]).all()
        assert topk[b].tolist() == T.topk_index_order(scores[b], k).tolist()
