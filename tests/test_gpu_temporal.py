"""GPU temporal pruning step against the oracle's replay filter.

For one decode transition (previous step -> current step with a few appended
keys and an AR(1) query drift), the GPU step's decisions must equal the
oracle's ``run_filter`` (reference replay.py:172-222, with the ``wave``
refresh schedule) fed the same inputs: the dense GPU scores of the current
step, the previous step's block maxima and top-k, the absolute margin and the
scan order.  Kept blocks and the number of keys scored must match exactly;
evaluated keys carry the dense scores bit for bit; the top-k is the stable
top-k over the evaluated keys.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsa_amd import decode, temporal
from oracle import replay as R
from oracle import topk as T

pytestmark = pytest.mark.gpu


def transition(batch, prev_length, length, seed, hot=0.01, rho=0.95):
    gen = torch.Generator().manual_seed(seed)
    q_prev = torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)
    q_cur = rho * q_prev + math.sqrt(1 - rho * rho) * torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)
    w = torch.randn(batch, 64, generator=gen) / 8
    keys = torch.randn(batch, length, 128, generator=gen)
    n_hot = max(1, round(hot * length))
    for b in range(batch):
        keys[b, torch.randperm(length, generator=gen)[:n_hot]] *= 4
    return q_prev.to(torch.bfloat16), q_cur.to(torch.bfloat16), w, keys.to(torch.bfloat16)


CASES = [
    # block, method, scan order, wave, prev length, length, k
    (16, "dynamic", "previous_hot", 64, 3000, 3003, 128),
    (32, "dynamic", "upper_hot", 16, 3000, 3003, 128),
    (64, "static", "address", 0, 4096, 4100, 256),
    (64, "static_hot_first", "previous_hot", 0, 4096, 4100, 256),
    (64, "dynamic", "previous_hot", 1, 2048, 2048, 128),
    (64, "dynamic", "previous_hot", 32, 16384, 16385, 2048),
    (128, "dynamic", "address", 8, 5000, 5001, 300),
    # the C3 length (16384 -> 16385 keys, K=2048) at the other block sizes
    (16, "dynamic", "previous_hot", 64, 16384, 16385, 2048),
    (32, "dynamic", "upper_hot", 16, 16384, 16385, 2048),
    (128, "dynamic", "address", 8, 16384, 16385, 2048),
    (16, "static_hot_first", "previous_hot", 0, 16384, 16385, 2048),
]


@pytest.mark.parametrize("block,method,order,wave,prev_length,length,k", CASES)
def test_temporal_step_matches_replay_filter(device, block, method, order, wave, prev_length, length, k) -> None:
    print(f"temporal bs={block} {method}/{order} wave={wave} L={prev_length}->{length} k={k}", flush=True)
    batch = 3
    q_prev, q_cur, w, keys = transition(batch, prev_length, length, seed=block * 7 + length)
    q_prev, q_cur, w, keys = q_prev.to(device), q_cur.to(device), w.to(device), keys.to(device)
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys[:, :prev_length].contiguous(), k, return_scores=True)
    prev_max = temporal.block_max(prev_scores, block)
    dense = decode.indexer_topk(q_cur, w, keys, k, return_scores=True)[1].cpu().numpy()
    spread = float(prev_scores.std())
    gamma = torch.full((batch,), 0.15 * spread, device=device)
    step = temporal.temporal_step(q_cur, w, keys, prev_max, prev_length, prev_topk, gamma, block_size=block,
                                  method=method, scan_order=order, wave=max(wave, 1))
    got_scores = step.scores.cpu().numpy()
    got_kept = step.evaluated_blocks.cpu().numpy()
    got_qk = step.qk_scored.cpu().numpy()
    got_topk = step.topk.cpu().numpy()
    prev_max_h = prev_max.cpu().double().numpy()
    seeds = prev_topk.cpu().numpy()
    schedule, dynamic, _ = R.method_schedule(method, order)
    blocks = math.ceil(length / block)
    pruned_any = False
    for b in range(batch):
        previous_max = np.full(blocks, -np.inf)
        previous_max[: prev_max_h.shape[1]] = prev_max_h[b]
        upper = R.upper_bounds(previous_max, float(gamma[b]), prev_length, length, block)
        hot = np.zeros(blocks, dtype=bool)
        hot[seeds[b] // block] = True
        scan = R.block_scan_order(schedule, upper, R.block_maxima(dense[b], block), hot)
        current = dense[b].astype(np.float64)
        tau_seed = float(current[seeds[b]].min())
        trace = R.run_filter(current, seeds[b], k, block, upper, scan, dynamic=dynamic, fixed_threshold=tau_seed,
                             wave=wave if dynamic else 1)
        np.testing.assert_array_equal(got_kept[b], trace.kept, err_msg=f"row {b}: kept blocks")
        assert int(got_qk[b]) == trace.scored, (b, int(got_qk[b]), trace.scored)
        ev = trace.evaluated
        np.testing.assert_array_equal(got_scores[b][ev], dense[b][ev])
        assert np.isneginf(got_scores[b][~ev]).all()
        masked = np.where(ev, dense[b], -np.inf).astype(np.float32)
        assert got_topk[b].tolist() == T.topk_index_order(masked, k).tolist(), b
        pruned_any |= not trace.kept.all()
    if block <= 32 and method == "dynamic":  # small blocks' maxima sit near the cut: these cases must prune
        assert pruned_any, "the margin pruned nothing: the case does not exercise pruning"


def test_temporal_step_fp8(device) -> None:
    print("temporal fp8 keys", flush=True)
    batch, prev_length, length, k, block = 2, 8192, 8200, 512, 64
    q_prev, q_cur, w, keys = transition(batch, prev_length, length, seed=31)
    raw = keys.float()
    blocks128 = math.ceil(length / 128)
    scales = torch.stack([torch.stack([raw[b, j * 128 : (j + 1) * 128].abs().max() / 448 for j in range(blocks128)]) for b in range(batch)])
    keys8 = (raw / scales.repeat_interleave(128, dim=1)[:, :length, None]).to(torch.float8_e4m3fn)
    q_prev, q_cur, w, keys8, scales = q_prev.to(device), q_cur.to(device), w.to(device), keys8.to(device), scales.to(device)
    prev_scales = scales[:, : math.ceil(prev_length / 128)].contiguous()
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys8[:, :prev_length].contiguous(), k,
                                                 key_scales=prev_scales, return_scores=True)
    prev_max = temporal.block_max(prev_scores, block)
    dense = decode.indexer_topk(q_cur, w, keys8, k, key_scales=scales, return_scores=True)[1].cpu().numpy()
    gamma = 0.15 * float(prev_scores.std())
    step = temporal.temporal_step(q_cur, w, keys8, prev_max, prev_length, prev_topk, gamma, block_size=block,
                                  method="dynamic", scan_order="previous_hot", wave=16, key_scales=scales)
    seeds = prev_topk.cpu().numpy()
    for b in range(batch):
        blocks = math.ceil(length / block)
        previous_max = np.full(blocks, -np.inf)
        previous_max[: prev_max.shape[1]] = prev_max[b].cpu().double().numpy()
        upper = R.upper_bounds(previous_max, float(np.float32(gamma)), prev_length, length, block)
        hot = np.zeros(blocks, dtype=bool)
        hot[seeds[b] // block] = True
        scan = R.block_scan_order("previous_hot", upper, R.block_maxima(dense[b], block), hot)
        current = dense[b].astype(np.float64)
        trace = R.run_filter(current, seeds[b], k, block, upper, scan, dynamic=True,
                             fixed_threshold=float(current[seeds[b]].min()), wave=16)
        np.testing.assert_array_equal(step.evaluated_blocks[b].cpu().numpy(), trace.kept)
        assert int(step.qk_scored[b]) == trace.scored
        ev = trace.evaluated
        np.testing.assert_array_equal(step.scores[b].cpu().numpy()[ev], dense[b][ev])


@pytest.mark.parametrize("method,order,wave,gamma_sigma",
                         [("dynamic", "previous_hot", 64, -0.25), ("static", "address", 0, -3.0)])
def test_temporal_step_fp8_c5_length(device, method, order, wave, gamma_sigma) -> None:
    # The C5 length: 131072 fp8 keys (one appended), block 64 (2048 blocks),
    # K=2048, against the oracle's filter on the dense GPU scores.
    print(f"temporal fp8 C5 length {method}/{order} wave={wave}", flush=True)
    batch, prev_length, length, k, block = 2, 131071, 131072, 2048, 64
    q_prev, q_cur, w, keys = transition(batch, prev_length, length, seed=131)
    raw = keys.float()
    blocks128 = math.ceil(length / 128)
    scales = raw.reshape(batch, blocks128, 128 * 128).abs().amax(dim=2) / 448
    keys8 = (raw / scales.repeat_interleave(128, dim=1)[..., None]).to(torch.float8_e4m3fn)
    del raw
    q_prev, q_cur, w, keys8, scales = q_prev.to(device), q_cur.to(device), w.to(device), keys8.to(device), scales.to(device)
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys8[:, :prev_length].contiguous(), k,
                                                 key_scales=scales[:, : math.ceil(prev_length / 128)].contiguous(),
                                                 return_scores=True)
    prev_max = temporal.block_max(prev_scores, block)
    dense = decode.indexer_topk(q_cur, w, keys8, k, key_scales=scales, return_scores=True)[1].cpu().numpy()
    gamma = gamma_sigma * float(prev_scores.std())  # a negative margin, so that blocks are pruned
    step = temporal.temporal_step(q_cur, w, keys8, prev_max, prev_length, prev_topk, gamma, block_size=block,
                                  method=method, scan_order=order, wave=max(wave, 1), key_scales=scales)
    seeds = prev_topk.cpu().numpy()
    schedule, dynamic, _ = R.method_schedule(method, order)
    pruned_any = False
    for b in range(batch):
        blocks = math.ceil(length / block)
        previous_max = np.full(blocks, -np.inf)
        previous_max[: prev_max.shape[1]] = prev_max[b].cpu().double().numpy()
        upper = R.upper_bounds(previous_max, float(np.float32(gamma)), prev_length, length, block)
        hot = np.zeros(blocks, dtype=bool)
        hot[seeds[b] // block] = True
        scan = R.block_scan_order(schedule, upper, R.block_maxima(dense[b], block), hot)
        current = dense[b].astype(np.float64)
        trace = R.run_filter(current, seeds[b], k, block, upper, scan, dynamic=dynamic,
                             fixed_threshold=float(current[seeds[b]].min()), wave=wave if dynamic else 1)
        np.testing.assert_array_equal(step.evaluated_blocks[b].cpu().numpy(), trace.kept)
        assert int(step.qk_scored[b]) == trace.scored
        ev = trace.evaluated
        np.testing.assert_array_equal(step.scores[b].cpu().numpy()[ev], dense[b][ev])
        masked = np.where(ev, dense[b], -np.inf).astype(np.float32)
        assert step.topk[b].cpu().numpy().tolist() == T.topk_index_order(masked, k).tolist(), b
        pruned_any |= not trace.kept.all()
    assert pruned_any, "the negative margin pruned nothing"


STATIC_CASES = [
    # block, gamma_sigma (negative: blocks are pruned), prev length, length, k, dtype
    (16, -1.0, 16384, 16385, 2048, torch.bfloat16),
    (16, -4.0, 16384, 16385, 2048, torch.bfloat16),
    (32, -3.0, 16384, 16385, 2048, torch.float16),
    (64, -3.0, 5000, 5003, 300, torch.bfloat16),
    (128, -5.0, 16384, 16400, 2048, torch.bfloat16),
    (64, 0.25, 16384, 16385, 2048, torch.bfloat16),
    (16, -3.0, 100, 100, 40, torch.bfloat16),
]


@pytest.mark.parametrize("block,gamma_sigma,prev_length,length,k,dtype", STATIC_CASES)
def test_static_step_paths_agree(device, monkeypatch, block, gamma_sigma, prev_length, length, k, dtype) -> None:
    # The static filter (fixed seed threshold) runs as one cooperative scoring
    # launch + the list select; DSA_AMD_TEMPORAL_PATH=launch runs it on the
    # prep / seed / block / histogram-select launches.  Both must equal the
    # oracle's filter, and each other bit for bit, also when pruned blocks
    # hold seeds.
    print(f"static paths bs={block} gs={gamma_sigma} L={prev_length}->{length} k={k} {dtype}", flush=True)
    batch = 3
    q_prev, q_cur, w, keys = transition(batch, prev_length, length, seed=block + length)
    q_prev, q_cur, keys = q_prev.to(dtype), q_cur.to(dtype), keys.to(dtype)
    q_prev, q_cur, w, keys = q_prev.to(device), q_cur.to(device), w.to(device), keys.to(device)
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys[:, :prev_length].contiguous(), k, return_scores=True)
    prev_max = temporal.block_max(prev_scores, block)
    dense = decode.indexer_topk(q_cur, w, keys, k, return_scores=True)[1].cpu().numpy()
    gamma = torch.full((batch,), gamma_sigma * float(prev_scores.std()), device=device)

    def run():
        s = temporal.temporal_step(q_cur, w, keys, prev_max, prev_length, prev_topk, gamma, block_size=block,
                                   method="static")
        assert s.waits_given_up.cpu().numpy().tolist() == [0] * batch, "a wait gave up"
        return (s.scores.cpu().numpy(), s.evaluated_blocks.cpu().numpy(), s.qk_scored.cpu().numpy(),
                s.topk.cpu().numpy())

    fused = run()
    monkeypatch.setenv("DSA_AMD_TEMPORAL_PATH", "launch")
    launch = run()
    monkeypatch.delenv("DSA_AMD_TEMPORAL_PATH")
    again = run()  # the fused path a second time on the same workspace (a new generation)
    for name, a, b, c in zip(("scores", "kept", "qk", "topk"), fused, launch, again):
        np.testing.assert_array_equal(a, b, err_msg=f"fused vs launch path: {name}")
        np.testing.assert_array_equal(a, c, err_msg=f"fused, second call: {name}")
    scores, kept, qk, topk = fused
    seeds = prev_topk.cpu().numpy()
    blocks = math.ceil(length / block)
    seeds_in_pruned = 0
    for b in range(batch):
        previous_max = np.full(blocks, -np.inf)
        previous_max[: prev_max.shape[1]] = prev_max[b].cpu().double().numpy()
        upper = R.upper_bounds(previous_max, float(gamma[b]), prev_length, length, block)
        scan = R.block_scan_order("address", upper, R.block_maxima(dense[b], block), np.zeros(blocks, dtype=bool))
        current = dense[b].astype(np.float64)
        trace = R.run_filter(current, seeds[b], k, block, upper, scan, dynamic=False,
                             fixed_threshold=float(current[seeds[b]].min()), wave=1)
        np.testing.assert_array_equal(kept[b], trace.kept, err_msg=f"row {b}: kept blocks")
        assert int(qk[b]) == trace.scored, (b, int(qk[b]), trace.scored)
        ev = trace.evaluated
        np.testing.assert_array_equal(scores[b][ev], dense[b][ev])
        assert np.isneginf(scores[b][~ev]).all()
        masked = np.where(ev, dense[b], -np.inf).astype(np.float32)
        assert topk[b].tolist() == T.topk_index_order(masked, k).tolist(), b
        seeds_in_pruned += int((~trace.kept[seeds[b] // block]).sum())
    if gamma_sigma <= -3.0:
        assert not kept.all(), "the negative margin pruned nothing"
    if gamma_sigma <= -4.0:  # below the seeds' own drift: blocks holding seeds are pruned too
        assert seeds_in_pruned > 0, "no pruned block holds a seed"


def test_static_step_reports_given_up_waits(device, monkeypatch) -> None:
    # The host makes every fused workgroup's bounded wait for its row's seed
    # minima give up at once (a spin limit of 0 polls): the kernel still ends
    # normally, each workgroup keeps every block of its chunk, and the step
    # reports the given-up waits.  The documented superset is then the dense
    # step: every block kept, every key scored with its dense score, and the
    # dense top-k.  The next call, with the default limit, is the filter's
    # exact step again and reports none.
    print("static step: given-up waits forced from the host", flush=True)
    batch, prev_length, length, k, block = 4, 16384, 16385, 2048, 64
    q_prev, q_cur, w, keys = transition(batch, prev_length, length, seed=77)
    q_prev, q_cur, w, keys = q_prev.to(device), q_cur.to(device), w.to(device), keys.to(device)
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys[:, :prev_length].contiguous(), k, return_scores=True)
    prev_max = temporal.block_max(prev_scores, block)
    dense = decode.indexer_topk(q_cur, w, keys, k, return_scores=True)[1].cpu().numpy()
    gamma = torch.full((batch,), -3.0 * float(prev_scores.std()), device=device)

    def run():
        return temporal.temporal_step(q_cur, w, keys, prev_max, prev_length, prev_topk, gamma, block_size=block,
                                      method="static")

    monkeypatch.setenv("DSA_AMD_STATIC_SPIN_LIMIT", "0")
    forced = run()
    monkeypatch.delenv("DSA_AMD_STATIC_SPIN_LIMIT")
    gave_up = forced.waits_given_up.cpu().numpy()
    assert (gave_up > 0).all(), gave_up
    assert forced.evaluated_blocks.cpu().numpy().all()
    assert forced.qk_scored.cpu().numpy().tolist() == [length] * batch
    np.testing.assert_array_equal(forced.scores.cpu().numpy(), dense)
    for b in range(batch):
        assert forced.topk[b].cpu().numpy().tolist() == T.topk_index_order(dense[b], k).tolist(), b

    exact = run()
    assert exact.waits_given_up.cpu().numpy().tolist() == [0] * batch
    kept = exact.evaluated_blocks.cpu().numpy()
    assert not kept.all(), "the negative margin pruned nothing"
    seeds = prev_topk.cpu().numpy()
    blocks = math.ceil(length / block)
    for b in range(batch):
        previous_max = np.full(blocks, -np.inf)
        previous_max[: prev_max.shape[1]] = prev_max[b].cpu().double().numpy()
        upper = R.upper_bounds(previous_max, float(gamma[b]), prev_length, length, block)
        scan = R.block_scan_order("address", upper, R.block_maxima(dense[b], block), np.zeros(blocks, dtype=bool))
        current = dense[b].astype(np.float64)
        trace = R.run_filter(current, seeds[b], k, block, upper, scan, dynamic=False,
                             fixed_threshold=float(current[seeds[b]].min()), wave=1)
        np.testing.assert_array_equal(kept[b], trace.kept, err_msg=f"row {b}: kept blocks")
        assert int(exact.qk_scored[b]) == trace.scored


@pytest.mark.parametrize("batch,prev_length,length,k,block,capacity", [
    (2, 5000, 5003, 300, 64, 8192),   # a view of a larger KV cache (key stride 8192 rows)
    (24, 700, 705, 700, 16, 705),     # many short rows; every previous key is a seed
    (1, 100, 100, 100, 32, 100),      # one row, one chunk, k = length
])
def test_static_step_cache_views_and_shapes(device, monkeypatch, batch, prev_length, length, k, block, capacity) -> None:
    print(f"static shapes B={batch} L={prev_length}->{length} k={k} bs={block} cap={capacity}", flush=True)
    q_prev, q_cur, w, cache = transition(batch, prev_length, capacity, seed=batch * 31 + length)
    q_prev, q_cur, w, cache = q_prev.to(device), q_cur.to(device), w.to(device), cache.to(device)
    view = cache[:, :length]
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, cache[:, :prev_length].contiguous(), k,
                                                 return_scores=True)
    prev_max = temporal.block_max(prev_scores, block)
    dense = decode.indexer_topk(q_cur, w, view.contiguous(), k, return_scores=True)[1].cpu().numpy()
    gamma = torch.full((batch,), -1.0 * float(prev_scores.std()), device=device)

    def run(keys):
        s = temporal.temporal_step(q_cur, w, keys, prev_max, prev_length, prev_topk, gamma, block_size=block,
                                   method="static")
        return [x.cpu().numpy() for x in (s.scores, s.evaluated_blocks, s.qk_scored, s.topk)]

    fused_view = run(view)
    fused_copy = run(view.contiguous())
    monkeypatch.setenv("DSA_AMD_TEMPORAL_PATH", "launch")
    launch_view = run(view)
    monkeypatch.delenv("DSA_AMD_TEMPORAL_PATH")
    for a, b, c in zip(fused_view, fused_copy, launch_view):
        np.testing.assert_array_equal(a, b)
        np.testing.assert_array_equal(a, c)
    scores, kept, qk, topk = fused_view
    seeds = prev_topk.cpu().numpy()
    blocks = math.ceil(length / block)
    for b in range(batch):
        previous_max = np.full(blocks, -np.inf)
        previous_max[: prev_max.shape[1]] = prev_max[b].cpu().double().numpy()
        upper = R.upper_bounds(previous_max, float(gamma[b]), prev_length, length, block)
        scan = R.block_scan_order("address", upper, R.block_maxima(dense[b], block), np.zeros(blocks, dtype=bool))
        current = dense[b].astype(np.float64)
        trace = R.run_filter(current, seeds[b], k, block, upper, scan, dynamic=False,
                             fixed_threshold=float(current[seeds[b]].min()), wave=1)
        np.testing.assert_array_equal(kept[b], trace.kept, err_msg=f"row {b}: kept blocks")
        assert int(qk[b]) == trace.scored, (b, int(qk[b]), trace.scored)
        ev = trace.evaluated
        np.testing.assert_array_equal(scores[b][ev], dense[b][ev])
        assert np.isneginf(scores[b][~ev]).all()
        masked = np.where(ev, dense[b], -np.inf).astype(np.float32)
        assert topk[b].tolist() == T.topk_index_order(masked, k).tolist(), b


DYNAMIC_CASES = [
    # block, scan order, wave, gamma_sigma, prev length, length, k, dtype, distinct keys (0: all distinct)
    (16, "previous_hot", 33, 0.25, 16384, 16385, 2048, torch.bfloat16, 0),
    (16, "address", 33, -0.5, 16384, 16385, 2048, torch.bfloat16, 0),
    (32, "upper_hot", 17, -1.0, 16384, 16385, 2048, torch.float16, 0),
    (64, "previous_hot", 1, -0.5, 4096, 4100, 256, torch.bfloat16, 0),
    (128, "address", 5, -1.0, 16384, 16400, 2048, torch.bfloat16, 0),
    (16, "address", 64, -1.0, 8000, 8003, 512, torch.bfloat16, 37),   # 37 distinct keys: scores tie in crowds
    (64, "previous_hot", 8, -2.0, 3000, 3000, 1000, torch.bfloat16, 5),
    # k = 4096 of 16K keys: a single round lists more keys than the replay's
    # LDS holds, so its sort spills to the workspace
    (16, "address", 64, -0.5, 16384, 16385, 4096, torch.bfloat16, 0),
]


@pytest.mark.parametrize("block,order,wave,gamma_sigma,prev_length,length,k,dtype,distinct", DYNAMIC_CASES)
def test_dynamic_step_paths_agree(device, monkeypatch, block, order, wave, gamma_sigma, prev_length, length, k,
                                  dtype, distinct) -> None:
    # The dynamic filter runs in rounds (wide scoring of the blocks above the
    # round's floor, then an exact replay per row); DSA_AMD_TEMPORAL_PATH=launch
    # runs the sequential scan (persistent per-row scan or per-wave launches).
    # Every round split must equal that path and the oracle's filter bit for
    # bit, also when scores tie in crowds around the threshold.
    print(f"dynamic paths bs={block} {order} W={wave} gs={gamma_sigma} L={length} k={k} {dtype} d={distinct}",
          flush=True)
    batch = 3
    q_prev, q_cur, w, keys = transition(batch, prev_length, length, seed=block * 3 + length + distinct)
    if distinct:
        keys = keys[:, torch.arange(length) % distinct]
    q_prev, q_cur, keys = q_prev.to(dtype), q_cur.to(dtype), keys.to(dtype)
    q_prev, q_cur, w, keys = q_prev.to(device), q_cur.to(device), w.to(device), keys.to(device)
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys[:, :prev_length].contiguous(), k, return_scores=True)
    prev_max = temporal.block_max(prev_scores, block)
    dense = decode.indexer_topk(q_cur, w, keys, k, return_scores=True)[1].cpu().numpy()
    gamma = torch.full((batch,), gamma_sigma * float(prev_scores.std()), device=device)

    def run(loads=None):
        s = temporal.temporal_step(q_cur, w, keys, prev_max, prev_length, prev_topk, gamma, block_size=block,
                                   method="dynamic", scan_order=order, wave=wave)
        if loads is not None:
            loads.append(temporal.keys_loaded(s, block).cpu().numpy())
        return [x.cpu().numpy() for x in (s.scores, s.evaluated_blocks, s.qk_scored, s.topk)]

    results = {}
    for splits in ("1", "0.25", "0.1,0.3,0.6"):
        monkeypatch.setenv("DSA_AMD_TEMPORAL_ROUNDS", splits)
        loads = []
        results[splits] = run(loads)
        # Key rows loaded: every evaluated key (seeds are loaded by the seed
        # pass, kept blocks by a round), at most the seeds and every key once.
        qk = results[splits][2]
        assert (loads[0] >= qk).all() and (loads[0] <= k + length).all(), (splits, loads[0], qk)
    monkeypatch.delenv("DSA_AMD_TEMPORAL_ROUNDS")
    monkeypatch.setenv("DSA_AMD_TEMPORAL_PATH", "launch")
    sequential = run()
    monkeypatch.delenv("DSA_AMD_TEMPORAL_PATH")
    for splits, got in results.items():
        for name, a, b in zip(("scores", "kept", "qk", "topk"), got, sequential):
            np.testing.assert_array_equal(a, b, err_msg=f"rounds {splits} vs the sequential scan: {name}")
    scores, kept, qk, topk = sequential
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
        masked = np.where(ev, dense[b], -np.inf).astype(np.float32)
        assert topk[b].tolist() == T.topk_index_order(masked, k).tolist(), b
    if not distinct:
        assert not kept.all(), "the margin pruned nothing: the case does not exercise the replay"


@pytest.mark.parametrize("gamma_sigma", [-2.0, 0.5])
def test_dynamic_step_topk_with_invalid_and_repeated_seeds(device, monkeypatch, gamma_sigma) -> None:
    # The rounds path takes the step's top-k from its last replay, whose k-th
    # largest evaluated score is checked against the scores row; seeds that
    # are out of range or repeated make the run's k-th largest differ from the
    # row's, so the row's own k-th largest is found instead.  Every output must equal the
    # sequential scan's (histogram select), and the top-k must be the stable
    # top-k of the returned scores row, -inf keys included.
    print(f"dynamic top-k with invalid/repeated seeds gs={gamma_sigma}", flush=True)
    batch, prev_length, length, k, block, wave = 2, 4096, 4100, 256, 16, 8
    q_prev, q_cur, w, keys = transition(batch, prev_length, length, seed=4242)
    q_prev, q_cur, w, keys = q_prev.to(device), q_cur.to(device), w.to(device), keys.to(device)
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys[:, :prev_length].contiguous(), k, return_scores=True)
    prev_max = temporal.block_max(prev_scores, block)
    seeds = prev_topk.clone()
    seeds[0, :40] = -1                   # no key
    seeds[0, 40:80] = seeds[0, 80:120]   # the same keys twice
    seeds[1, 10:] = length + 5           # past the row: ten valid seeds
    gamma = torch.full((batch,), gamma_sigma * float(prev_scores.std()), device=device)

    def run():
        s = temporal.temporal_step(q_cur, w, keys, prev_max, prev_length, seeds, gamma, block_size=block,
                                   method="dynamic", scan_order="address", wave=wave)
        return [x.cpu().numpy() for x in (s.scores, s.evaluated_blocks, s.qk_scored, s.topk)]

    results = {}
    for splits in ("1", "0.25"):
        monkeypatch.setenv("DSA_AMD_TEMPORAL_ROUNDS", splits)
        results[splits] = run()
    monkeypatch.delenv("DSA_AMD_TEMPORAL_ROUNDS")
    monkeypatch.setenv("DSA_AMD_TEMPORAL_PATH", "launch")
    sequential = run()
    monkeypatch.delenv("DSA_AMD_TEMPORAL_PATH")
    for splits, got in results.items():
        for name, a, b in zip(("scores", "kept", "qk", "topk"), got, sequential):
            np.testing.assert_array_equal(a, b, err_msg=f"rounds {splits} vs the sequential scan: {name}")
    scores, _, qk, topk = sequential
    for b in range(batch):
        assert topk[b].tolist() == T.topk_index_order(scores[b], k).tolist(), b
        assert int(qk[b]) == int(np.isfinite(scores[b]).sum()), b


def test_dynamic_step_keys_loaded_accounting(device, monkeypatch) -> None:
    # Key rows a dynamic step loads on the rounds path: the seeds, then per
    # round every non-seed key of the blocks whose bound clears the round's
    # floor (the k-th largest evaluated score at the round's start: the seed
    # threshold for the first round).  Recomputed on the host from the
    # oracle's filter run up to each round boundary.
    print("dynamic keys loaded accounting", flush=True)
    batch, prev_length, length, k, block, wave = 2, 8000, 8003, 512, 16, 16
    q_prev, q_cur, w, keys = transition(batch, prev_length, length, seed=77)
    q_prev, q_cur, w, keys = q_prev.to(device), q_cur.to(device), w.to(device), keys.to(device)
    prev_topk, prev_scores = decode.indexer_topk(q_prev, w, keys[:, :prev_length].contiguous(), k, return_scores=True)
    prev_max = temporal.block_max(prev_scores, block)
    dense = decode.indexer_topk(q_cur, w, keys, k, return_scores=True)[1].cpu().numpy()
    gamma = torch.full((batch,), -0.5 * float(prev_scores.std()), device=device)
    seeds = prev_topk.cpu().numpy()
    blocks = math.ceil(length / block)
    groups = math.ceil(blocks / wave)
    for splits, fractions in (("1", []), ("0.25", [0.25])):
        monkeypatch.setenv("DSA_AMD_TEMPORAL_ROUNDS", splits)
        step = temporal.temporal_step(q_cur, w, keys, prev_max, prev_length, prev_topk, gamma, block_size=block,
                                      method="dynamic", scan_order="previous_hot", wave=wave)
        got = temporal.keys_loaded(step, block).cpu().numpy()
        cuts = [0] + [int(f * groups + 0.5) for f in fractions] + [groups]
        for b in range(batch):
            previous_max = np.full(blocks, -np.inf)
            previous_max[: prev_max.shape[1]] = prev_max[b].cpu().double().numpy()
            upper = R.upper_bounds(previous_max, float(gamma[b]), prev_length, length, block)
            hot = np.zeros(blocks, dtype=bool)
            hot[seeds[b] // block] = True
            order = R.block_scan_order("previous_hot", upper, R.block_maxima(dense[b], block), hot)
            current = dense[b].astype(np.float64)
            tau_seed = float(current[seeds[b]].min())
            is_seed = np.zeros(length, dtype=bool)
            is_seed[seeds[b]] = True
            want = k
            for r in range(len(cuts) - 1):
                lo, hi = cuts[r] * wave, min(cuts[r + 1] * wave, blocks)
                if r == 0:
                    floor = tau_seed
                else:  # the k-th largest evaluated score after the scan's first lo positions
                    trace = R.run_filter(current, seeds[b], k, block, upper, order[:lo], dynamic=True,
                                         fixed_threshold=tau_seed, wave=wave)
                    floor = trace.threshold_final
                for blk in order[lo:hi]:
                    if not upper[blk] < np.float32(floor):
                        keys_b = np.arange(blk * block, min(length, (blk + 1) * block))
                        want += int((~is_seed[keys_b]).sum())
            assert int(got[b]) == want, (splits, b, int(got[b]), want)
    monkeypatch.delenv("DSA_AMD_TEMPORAL_ROUNDS")
