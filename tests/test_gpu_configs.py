"""Full-size parity cases of the BASELINE configurations other than the bench's.

C4 (prefill): T=4096 queries x L=4096 causal keys, bf16 ~ N(0,1)/sqrt(128),
64x128 indexer, fp32 accumulation, per-query top-K=512 under the causal mask
(rows with fewer than 512 visible keys return them all, padded with -1).
C5 (long-context fp8 decode): B=4, L=131072 fp8 e4m3fn keys with one fp32
scale per 128-key block, keys drawn around 10 Gaussian topic centroids,
bf16 queries, top-K=2048.

Index sets are checked bit-exactly against stable_topk of the kernel's own
scores (every row); the scores against the float64 oracle on sampled keys.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsa_amd import decode, metrics, sidecar
from oracle import scores as S
from oracle import topk as T

pytestmark = pytest.mark.gpu


def _check_scores(got, q, w, keys, idx) -> None:
    """Kernel scores at key positions idx against the float64 closed form."""

    ref = S.relu_index_score(q, keys[idx], w)
    scale = S.abs_weight_scale(q, keys[idx], w)
    assert np.all(np.abs(got[idx] - ref) <= 1e-5 * scale + 1e-6)


def test_c4_prefill_causal_top512(device) -> None:
    print("C4 prefill T=4096 L=4096 causal top-512", flush=True)
    gen = torch.Generator().manual_seed(1582)
    t, length, k = 4096, 4096, 512
    q = (torch.randn(1, t, 64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16)
    w = torch.randn(1, t, 64, generator=gen) / 8
    keys = (torch.randn(1, length, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16)
    scores = sidecar.score_encoded(q.to(device), w.to(device), keys.to(device), causal=True)[0]
    visible = torch.arange(1, t + 1, dtype=torch.int32, device=device)  # query i sees keys 0..i
    idx = metrics.topk(scores, k, sorted=False, row_lengths=visible).cpu().numpy()
    host = scores.cpu().numpy()
    for row in range(t):
        n = row + 1
        want = T.topk_index_order(host[row, :n], min(k, n))
        assert idx[row, : want.size].tolist() == want.tolist(), row
        assert (idx[row, want.size :] == -1).all(), row
        assert np.isneginf(host[row, n:]).all(), row
    rng = np.random.default_rng(4)
    kf = keys[0].float().numpy()
    for row in (0, 1, 511, 512, 2047, 4095):
        cols = rng.choice(row + 1, size=min(row + 1, 256), replace=False)
        _check_scores(host[row], q[0, row].float().numpy(), w[0, row].numpy(), kf, cols)


def test_c5_fp8_long_context_top2048(device) -> None:
    print("C5 fp8 B=4 L=131072 top-2048", flush=True)
    gen = torch.Generator().manual_seed(1582)
    batch, length, k = 4, 131072, 2048
    q = (torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16)
    w = torch.randn(batch, 64, generator=gen) / 8
    centroids = torch.randn(batch, 10, 128, generator=gen)
    topic = torch.randint(0, 10, (batch, length), generator=gen)
    raw = (torch.gather(centroids, 1, topic[..., None].expand(-1, -1, 128)) + torch.randn(batch, length, 128, generator=gen)) / math.sqrt(2)
    blocks = length // 128
    scales = raw.reshape(batch, blocks, 128 * 128).abs().amax(dim=2) / 448.0
    keys8 = (raw / scales.repeat_interleave(128, dim=1)[..., None]).to(torch.float8_e4m3fn)
    del raw
    idx, scores = decode.indexer_topk(q.to(device), w.to(device), keys8.to(device), k, key_scales=scales.to(device), return_scores=True)
    idx = idx.cpu().numpy()
    host = scores.cpu().numpy()
    rng = np.random.default_rng(5)
    for b in range(batch):
        assert idx[b].tolist() == T.topk_index_order(host[b], k).tolist(), b
        cols = np.concatenate([idx[b][:256], rng.choice(length, size=1024, replace=False)])
        deq = S.dequantize_fp8_blocks(keys8[b : b + 1], scales[b : b + 1])[0]
        _check_scores(host[b], q[b].float().numpy(), w[b].numpy(), deq, cols)
