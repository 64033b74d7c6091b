"""GPU own-trajectory step against the oracle's ``replay_step`` (own mode).

A few decode steps of a growing context (one key appended per step, AR(1)
query drift) run twice: on the GPU through ``approx_step``, which scores only
what the policy keeps and advances the device metadata, and in the oracle
(reference approx.py:129-364, with the ``wave`` refresh schedule) fed the
dense GPU scores of each step.  Refreshed blocks, keys scored, the
approximate top-k set and every metadata array (last max, EMA, volatility,
age, cold streak) must match exactly at every step.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsa_amd import approx, decode
from oracle import approx as A

pytestmark = pytest.mark.gpu


def trajectory(batch, length, steps, seed, rho=0.95):
    gen = torch.Generator().manual_seed(seed)
    q = [torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)]
    for _ in range(steps):
        q.append(rho * q[-1] + math.sqrt(1 - rho * rho) * torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128))
    w = torch.randn(batch, 64, generator=gen) / 8
    keys = torch.randn(batch, length + steps, 128, generator=gen)
    hot = torch.rand(batch, length + steps, generator=gen) < 0.01
    keys[hot] *= 4
    return [x.to(torch.bfloat16) for x in q], w, keys.to(torch.bfloat16)


POLICIES = [
    # policy, block size, wave, gamma in units of the first step's score std
    (A.ApproxPolicy(name="static"), 64, 1, 0.1),
    (A.ApproxPolicy(name="dynamic_address", dynamic_threshold=True), 32, 1, 0.0),
    (A.ApproxPolicy(name="dynamic_previous_max", dynamic_threshold=True, order="previous_max"), 16, 8, -0.2),
    (A.ApproxPolicy(name="streak2_bucket8", dynamic_threshold=True, order="bucket8", cold_streak=2), 64, 4, -0.5),
    (
        A.ApproxPolicy(name="ema_bucket8_age8", dynamic_threshold=True, order="bucket8", risk_model="ema",
                       ema_alpha=0.9, volatility_lambda=2.0, age_cap=8),
        32, 16, -0.3,
    ),
    (
        # cold_streak=0: at k=256 of 4000 keys every 128-key block holds a
        # top-k key, so the default streak would force every block
        A.ApproxPolicy(name="recent_slope", dynamic_threshold=True, order="bucket16", recent_window=100,
                       age_slope=0.01, refresh_interval=4, cold_streak=0),
        128, 2, -1.0,
    ),
]


def to_device_policy(policy: A.ApproxPolicy, gamma: float) -> approx.ApproxPolicy:
    fields = {f: getattr(policy, f) for f in approx.ApproxPolicy.__dataclass_fields__}
    fields["gamma"] = gamma
    return approx.ApproxPolicy(**fields)


@pytest.mark.parametrize("policy,block,wave,gamma_sigma", POLICIES, ids=[p[0].name for p in POLICIES])
def test_approx_step_matches_oracle_trajectory(device, policy, block, wave, gamma_sigma) -> None:
    run_trajectory(device, policy, block, wave, gamma_sigma, batch=2, length=4000, steps=6, k=256,
                   seed=block + 17 * wave)


C3_POLICIES = [
    (A.ApproxPolicy(name="c3_dynamic_previous_max", dynamic_threshold=True, order="previous_max", cold_streak=0),
     64, 4, -0.3),
    (A.ApproxPolicy(name="c3_ema_bucket8", dynamic_threshold=True, order="bucket8", risk_model="ema", ema_alpha=0.9,
                    volatility_lambda=2.0, age_cap=8, cold_streak=0), 32, 16, -0.3),
]


@pytest.mark.parametrize("policy,block,wave,gamma_sigma", C3_POLICIES, ids=[p[0].name for p in C3_POLICIES])
def test_approx_step_c3_shape_trajectory(device, policy, block, wave, gamma_sigma) -> None:
    # The C3 replay shape: B=4 sequences from L=16384, K=2048, 20 own-trajectory
    # steps with the state carried on the device from step 0.
    run_trajectory(device, policy, block, wave, gamma_sigma, batch=4, length=16384, steps=20, k=2048, seed=4242)


def test_approx_step_c5_length_trajectory(device) -> None:
    # The C5 length (131072 keys, block 64, 96-block groups): the dynamic scan
    # runs in three rounds, with the policy's risk as the bound.
    policy = A.ApproxPolicy(name="c5_dynamic_previous_max", dynamic_threshold=True, order="previous_max",
                            cold_streak=0)
    run_trajectory(device, policy, 64, 96, -0.3, batch=2, length=131069, steps=3, k=2048, seed=5150)


def run_trajectory(device, policy, block, wave, gamma_sigma, *, batch, length, steps, k, seed) -> None:
    print(f"approx {policy.name} bs={block} wave={wave} gamma={gamma_sigma}sigma B={batch} L={length} "
          f"steps={steps} k={k}", flush=True)
    qs, w, keys = trajectory(batch, length, steps, seed=seed)
    w, keys = w.to(device), keys.to(device)
    _, scores0 = decode.indexer_topk(qs[0].to(device), w, keys[:, :length].contiguous(), k, return_scores=True)
    gamma = float(gamma_sigma * scores0.std())
    gpu_policy = to_device_policy(policy, gamma)
    cpu_policy = policy.with_gamma(gamma)
    state = approx.initialize_state(scores0, k=k, block_size=block, capacity=length + steps)
    host0 = scores0.cpu().numpy()
    oracle = [A.initialize_state(host0[b], k=k, block_size=block) for b in range(batch)]
    got = state.host()
    for b in range(batch):
        for field in ("last_max", "ema", "volatility", "age", "cold_streak"):
            np.testing.assert_array_equal(got[field][b], getattr(oracle[b], field), err_msg=f"init {field}")
        assert set(got["topk"][b].tolist()) == set(oracle[b].topk.tolist())
    skipped = 0
    for t in range(1, steps + 1):
        cur = length + t
        q = qs[t].to(device)
        dense = decode.indexer_topk(q, w, keys[:, :cur].contiguous(), k, return_scores=True)[1].cpu().numpy()
        step = approx.approx_step(state, q, w, keys[:, :cur], policy=gpu_policy, step=t, wave=wave)
        kept = step.evaluated_blocks.cpu().numpy()
        qk = step.qk_scored.cpu().numpy()
        top = step.topk.cpu().numpy()
        scores = step.scores.cpu().numpy()
        got = state.host()
        for b in range(batch):
            oracle[b], metrics, details = A.replay_step(
                oracle[b], dense[b], policy=cpu_policy, k=k, block_size=block, step=t, previous_length=cur - 1,
                wave=wave,
            )
            where = f"step {t} row {b}"
            refreshed = np.zeros(kept.shape[1], dtype=bool)
            refreshed[details["refreshed_blocks"]] = True
            np.testing.assert_array_equal(kept[b], refreshed, err_msg=f"{where}: refreshed blocks")
            assert int(qk[b]) == metrics["qk_scored"], where
            assert sorted(top[b].tolist()) == sorted(details["approximate"].tolist()), where
            ev = details["evaluated"]
            np.testing.assert_array_equal(scores[b][ev], dense[b][ev], err_msg=where)
            for field in ("last_max", "ema", "volatility", "age", "cold_streak"):
                np.testing.assert_array_equal(got[field][b], getattr(oracle[b], field), err_msg=f"{where}: {field}")
            skipped += metrics["blocks_skipped"]
    if gamma_sigma < 0:
        assert skipped > 0, "the policy skipped nothing: the case does not exercise pruning"


def test_approx_rejects_runtime_illegal_requests(device) -> None:
    scores = torch.randn(1, 512, device=device)
    state = approx.initialize_state(scores, k=16, block_size=64)
    q = torch.zeros(1, 64, 128, device=device, dtype=torch.bfloat16)
    w = torch.zeros(1, 64, device=device)
    keys = torch.zeros(1, 600, 128, device=device, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="oracle_current"):
        approx.approx_step(state, q, w, keys[:, :512], policy=approx.ApproxPolicy("o", order="oracle_current"), step=1)
    with pytest.raises(ValueError, match="capacity"):
        approx.approx_step(state, q, w, keys, policy=approx.ApproxPolicy("s"), step=1)
