"""GPU parity of the H8 / masked / progressive kernels.

Ports the reference's GPU tests (reference tests/test_progressive_kernel.py:
131-197) and checks every block size, ragged tails and the compact layout
against the kernel-semantics oracle (oracle.scores.kernel_*).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsa_amd.progressive_kernel import (
    dynamic_head_ids,
    full_scores_triton,
    h8_block_max_triton,
    masked_full_scores_triton,
    progressive_scores_triton,
    split_head_ids,
    two_pass_scores_triton,
)
from oracle import scores as S

pytestmark = pytest.mark.gpu


def cuda_inputs(length: int, device):
    gen = torch.Generator().manual_seed(1582)
    queries = (torch.randn(64, 128, generator=gen) * 0.1).to(torch.bfloat16)
    weights = torch.randn(64, generator=gen)
    keys = (torch.randn(length, 128, generator=gen) * 0.1).to(torch.bfloat16)
    return queries.to(device), weights.to(device), keys.to(device)


def test_progressive_all_promoted_matches_full_kernel(device) -> None:
    queries, weights, keys = cuda_inputs(257, device)
    direct = torch.zeros(math.ceil(len(keys) / 64), device=device, dtype=torch.int8)
    result = progressive_scores_triton(queries, weights, keys, dynamic_head_ids(weights.cpu()), direct, -math.inf)
    expected = full_scores_triton(queries, weights, keys)
    torch.testing.assert_close(result.scores, expected, rtol=1e-5, atol=1e-5)
    assert result.accepted_blocks.bool().all()


def test_progressive_direct_and_rejected_blocks(device) -> None:
    queries, weights, keys = cuda_inputs(128, device)
    direct = torch.tensor([1, 0], device=device, dtype=torch.int8)
    result = progressive_scores_triton(queries, weights, keys, torch.arange(8), direct, math.inf)
    expected = full_scores_triton(queries, weights, keys)
    torch.testing.assert_close(result.scores[:64], expected[:64], rtol=1e-5, atol=1e-5)
    assert torch.isneginf(result.scores[64:]).all()


def test_two_pass_matches_fused_decisions(device) -> None:
    queries, weights, keys = cuda_inputs(256, device)
    direct = torch.tensor([1, 0, 0, 1], device=device, dtype=torch.int8)
    heads = dynamic_head_ids(weights.cpu())
    probe = progressive_scores_triton(queries, weights, keys, heads, direct, math.inf)
    threshold = torch.quantile(probe.block_max[1:3], 0.5)
    fused = progressive_scores_triton(queries, weights, keys, heads, direct, threshold)
    two_pass = two_pass_scores_triton(queries, weights, keys, heads, direct, threshold)
    assert torch.equal(fused.accepted_blocks, two_pass.accepted_blocks)
    torch.testing.assert_close(fused.scores, two_pass.scores, rtol=1e-5, atol=1e-5)


def test_compact_output_matches_dense_candidates(device) -> None:
    queries, weights, keys = cuda_inputs(192, device)
    direct = torch.tensor([1, 0, 1], device=device, dtype=torch.int8)
    heads = dynamic_head_ids(weights.cpu())
    dense = progressive_scores_triton(queries, weights, keys, heads, direct, math.inf)
    compact = progressive_scores_triton(queries, weights, keys, heads, direct, math.inf, compact=True)
    assert compact.candidate_count == 128
    order = torch.argsort(compact.candidate_indices.long())
    indices = compact.candidate_indices[order].long()
    torch.testing.assert_close(compact.scores[order], dense.scores[indices])


def block_tolerance(scale: np.ndarray, block_size: int) -> np.ndarray:
    """Largest per-key score tolerance (1e-5 * S + 1e-6) of each block."""

    blocks = math.ceil(scale.size / block_size)
    padded = np.zeros(blocks * block_size)
    padded[: scale.size] = scale
    return 1e-5 * padded.reshape(blocks, block_size).max(axis=1) + 1e-6


@pytest.mark.parametrize("block_size", [16, 32, 64, 128])
@pytest.mark.parametrize("length", [100, 1000])
def test_kernels_match_oracle_semantics(device, block_size, length) -> None:
    print(f"progressive bs={block_size} L={length}", flush=True)
    gen = torch.Generator().manual_seed(block_size + length)
    q = (torch.randn(64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16)
    w = torch.randn(64, generator=gen) / 8
    k = torch.randn(length, 128, generator=gen).to(torch.bfloat16)
    blocks = math.ceil(length / block_size)
    direct = torch.rand(blocks, generator=gen) < 0.3
    selected, remaining = split_head_ids(dynamic_head_ids(w))
    qn, wn, kn = q.float().numpy(), w.numpy(), k.float().numpy()
    h8_part, h8_max = S.kernel_h8_block_max(qn, wn, kn, selected.numpy(), (~direct).numpy(), block_size)
    finite = np.sort(h8_max[np.isfinite(h8_max)])
    # Threshold halfway between two adjacent block maxima near the median, so
    # that fp32-vs-float64 rounding cannot flip a promotion decision.
    if finite.size >= 2:
        i = finite.size // 2 - 1
        threshold = float(0.5 * (finite[i] + finite[i + 1]))
        assert finite[i + 1] - finite[i] > 1e-4 * max(1.0, abs(threshold))
    else:
        threshold = 0.0
    ref, ref_acc, ref_max = S.kernel_progressive(qn, wn, kn, selected.numpy(), remaining.numpy(), direct.numpy(), threshold, block_size)
    scale = S.abs_weight_scale(qn, kn, wn)
    dq, dw, dk = q.to(device), w.to(device), k.to(device)

    part, maxima = h8_block_max_triton(dq, dw, dk, selected, ~direct, block_size=block_size)
    got_part = part.cpu().double().numpy()
    assert np.array_equal(np.isneginf(got_part), np.isneginf(h8_part))
    fin = np.isfinite(h8_part)
    assert np.all(np.abs(got_part[fin] - h8_part[fin]) <= 1e-5 * scale[fin] + 1e-6)
    got_max = maxima.cpu().double().numpy()
    assert np.array_equal(np.isneginf(got_max), np.isneginf(h8_max))
    # Block maxima (reference progressive_kernel.py:246): a maximum moves by at
    # most its block's largest per-key error, so each finite maximum is held
    # to the largest key tolerance of its block.
    tol = block_tolerance(scale, block_size)
    fin_b = np.isfinite(h8_max)
    assert np.all(np.abs(got_max[fin_b] - h8_max[fin_b]) <= tol[fin_b]), "h8 block maxima"

    result = progressive_scores_triton(dq, dw, dk, selected, direct, threshold, block_size=block_size)
    assert result.accepted_blocks.cpu().bool().numpy().tolist() == ref_acc.tolist()
    got = result.scores.cpu().double().numpy()
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert np.all(np.abs(got[fin] - ref[fin]) <= 1e-5 * scale[fin] + 1e-6)
    bm = result.block_max.cpu().double().numpy()
    assert np.array_equal(np.isneginf(bm), np.isneginf(ref_max))
    # ProgressiveResult.block_max (reference progressive_kernel.py:334): the H8
    # maximum of every screened block, -inf for direct blocks.
    fin_b = np.isfinite(ref_max)
    assert np.all(np.abs(bm[fin_b] - ref_max[fin_b]) <= tol[fin_b]), "progressive block_max"

    masked = masked_full_scores_triton(dq, dw, dk, result.accepted_blocks, block_size=block_size).cpu().double().numpy()
    ref_masked = S.kernel_masked_full(qn, wn, kn, ref_acc, block_size)
    assert np.array_equal(np.isneginf(masked), np.isneginf(ref_masked))
    assert np.all(np.abs(masked[fin] - ref_masked[fin]) <= 1e-5 * scale[fin] + 1e-6)

    compact = progressive_scores_triton(dq, dw, dk, selected, direct, threshold, block_size=block_size, compact=True)
    assert compact.candidate_count == int(np.isfinite(ref).sum())  # exact, ragged tail included
    idx = compact.candidate_indices.cpu().long()
    assert sorted(idx.tolist()) == np.flatnonzero(np.isfinite(ref)).tolist()
    assert torch.equal(compact.scores.cpu(), result.scores.cpu()[idx])


@pytest.mark.parametrize("block_size,length", [(16, 1000), (64, 1000), (128, 1000), (64, 131072)])
def test_fp8_keys_match_oracle_on_dequantised_keys(device, block_size, length) -> None:
    # fp8 e4m3fn keys with one fp32 scale per 128 keys: every kernel's scores
    # (partial or full) equal the oracle's on the dequantised keys, since the
    # ReLU commutes with a non-negative scale.  131072 keys is the C5 length.
    print(f"progressive fp8 bs={block_size} L={length}", flush=True)
    gen = torch.Generator().manual_seed(7 * block_size + length)
    q = (torch.randn(64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16)
    w = torch.randn(64, generator=gen) / 8
    raw = torch.randn(length, 128, generator=gen)
    nscale = math.ceil(length / 128)
    scales = torch.stack([raw[j * 128 : (j + 1) * 128].abs().max() / 448 for j in range(nscale)])
    k8 = (raw / scales.repeat_interleave(128)[:length, None]).to(torch.float8_e4m3fn)
    deq = S.dequantize_fp8_blocks(k8[None], scales[None])[0]
    blocks = math.ceil(length / block_size)
    direct = torch.rand(blocks, generator=gen) < 0.3
    selected, remaining = split_head_ids(dynamic_head_ids(w))
    qn, wn = q.float().numpy(), w.numpy()
    h8_part, h8_max = S.kernel_h8_block_max(qn, wn, deq, selected.numpy(), (~direct).numpy(), block_size)
    finite = np.sort(h8_max[np.isfinite(h8_max)])
    # A threshold in the widest gap between adjacent maxima near the median,
    # so that fp32-vs-float64 rounding cannot flip a promotion decision.
    mid = finite.size // 2
    lo = max(0, mid - 32)
    i = lo + int(np.argmax(np.diff(finite[lo : mid + 32])))
    threshold = float(0.5 * (finite[i] + finite[i + 1]))
    assert finite[i + 1] - finite[i] > 1e-4 * max(1.0, abs(threshold))
    ref, ref_acc, ref_max = S.kernel_progressive(qn, wn, deq, selected.numpy(), remaining.numpy(), direct.numpy(),
                                                 threshold, block_size)
    scale = S.abs_weight_scale(qn, deq, wn)
    tol = block_tolerance(scale, block_size)
    dq, dw, dk, ds = q.to(device), w.to(device), k8.to(device), scales.to(device)

    part, maxima = h8_block_max_triton(dq, dw, dk, selected, ~direct, block_size=block_size, key_scales=ds)
    got_part = part.cpu().double().numpy()
    assert np.array_equal(np.isneginf(got_part), np.isneginf(h8_part))
    fin = np.isfinite(h8_part)
    assert np.all(np.abs(got_part[fin] - h8_part[fin]) <= 1e-5 * scale[fin] + 1e-6)
    got_max = maxima.cpu().double().numpy()
    fin_b = np.isfinite(h8_max)
    assert np.array_equal(np.isneginf(got_max), ~fin_b)
    assert np.all(np.abs(got_max[fin_b] - h8_max[fin_b]) <= tol[fin_b]), "fp8 h8 block maxima"

    full = full_scores_triton(dq, dw, dk, key_scales=ds).cpu().double().numpy()
    ref_full = S.relu_index_score(qn, deq, wn)
    assert np.all(np.abs(full - ref_full) <= 1e-5 * scale + 1e-6)
    result = progressive_scores_triton(dq, dw, dk, selected, direct, threshold, block_size=block_size, key_scales=ds)
    assert result.accepted_blocks.cpu().bool().numpy().tolist() == ref_acc.tolist()
    got = result.scores.cpu().double().numpy()
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert np.all(np.abs(got[fin] - ref[fin]) <= 1e-5 * scale[fin] + 1e-6)
    bm = result.block_max.cpu().double().numpy()
    fin_b = np.isfinite(ref_max)
    assert np.array_equal(np.isneginf(bm), ~fin_b)
    assert np.all(np.abs(bm[fin_b] - ref_max[fin_b]) <= tol[fin_b]), "fp8 progressive block_max"
    two = two_pass_scores_triton(dq, dw, dk, selected, direct, threshold, block_size=block_size, key_scales=ds)
    assert torch.equal(two.accepted_blocks.cpu(), result.accepted_blocks.cpu())
    torch.testing.assert_close(two.scores.cpu(), result.scores.cpu(), rtol=1e-6, atol=1e-6)
    with pytest.raises(ValueError, match="key_scales"):
        progressive_scores_triton(dq, dw, dk, selected, direct, threshold, block_size=block_size)


def test_rejects_bad_masks_and_heads(device) -> None:
    queries, weights, keys = cuda_inputs(128, device)
    with pytest.raises(ValueError):
        progressive_scores_triton(queries, weights, keys, torch.arange(8), torch.zeros(3, dtype=torch.int8, device=device), 0.0)
    with pytest.raises(ValueError):
        progressive_scores_triton(queries, weights, keys, torch.arange(7), torch.zeros(2, dtype=torch.int8, device=device), 0.0)
    with pytest.raises(ValueError):
        h8_block_max_triton(queries, weights, keys, torch.arange(8), torch.zeros(5, dtype=torch.bool, device=device))
    with pytest.raises(ValueError):
        masked_full_scores_triton(queries, weights, keys, torch.zeros(1, dtype=torch.bool, device=device))
    with pytest.raises(ValueError):
        full_scores_triton(queries, weights, keys.float())


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("block_size,compact", [(16, False), (64, True), (128, False)])
def test_batched_progressive_equals_per_sequence(device, fp8, block_size, compact) -> None:
    # One launch over B sequences gives, row by row, exactly the single-
    # sequence kernel's result (scores, decisions, block maxima, compact
    # counts and candidates).
    from dsa_amd.progressive_kernel import progressive_scores_batched

    print(f"progressive batched fp8={fp8} bs={block_size} compact={compact}", flush=True)
    batch, length = 3, 1000
    gen = torch.Generator().manual_seed(block_size + 31 * fp8)
    q = (torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16)
    w = torch.randn(batch, 64, generator=gen) / 8
    raw = torch.randn(batch, length, 128, generator=gen)
    nscale = math.ceil(length / 128)
    scales = None
    if fp8:
        scales = torch.stack([torch.stack([raw[b, j * 128 : (j + 1) * 128].abs().max() / 448 for j in range(nscale)])
                              for b in range(batch)])
        keys = (raw / scales.repeat_interleave(128, dim=1)[:, :length, None]).to(torch.float8_e4m3fn)
    else:
        keys = raw.to(torch.bfloat16)
    blocks = math.ceil(length / block_size)
    direct = torch.rand(batch, blocks, generator=gen) < 0.3
    heads = torch.stack([dynamic_head_ids(w[b]) for b in range(batch)])
    thresholds = torch.tensor([0.05, -1.0, 0.2])
    dq, dw, dk = q.to(device), w.to(device), keys.to(device)
    ds = scales.to(device) if fp8 else None
    got = progressive_scores_batched(dq, dw, dk, heads, direct.to(device), thresholds.to(device),
                                     block_size=block_size, compact=compact, key_scales=ds)
    for b in range(batch):
        one = progressive_scores_triton(dq[b], dw[b], dk[b], heads[b], direct[b].to(device), float(thresholds[b]),
                                        block_size=block_size, compact=compact,
                                        key_scales=ds[b] if fp8 else None)
        assert torch.equal(got.accepted_blocks[b], one.accepted_blocks), b
        assert torch.equal(got.block_max[b], one.block_max), b
        if compact:
            n = int(got.candidate_count[b])
            assert n == one.candidate_count, b
            order_g = torch.argsort(got.candidate_indices[b, :n])
            order_o = torch.argsort(one.candidate_indices)
            assert torch.equal(got.candidate_indices[b, :n][order_g], one.candidate_indices[order_o]), b
            assert torch.equal(got.scores[b, :n][order_g], one.scores[order_o]), b
        else:
            assert torch.equal(got.scores[b], one.scores), b
