"""GPU verifier step and dim-sketch kernels against the oracle.

The live verifier step (``dsa_amd.verifier.verifier_step``) runs a few decode
steps of a growing context; the oracle's ``verifier_step`` (reference
verifier.py:173-392, restated in oracle/verifier.py and pinned there by the
reference's golden vectors) is fed, per step, the dense GPU scores and the
GPU's verifier scores of the cold keys.  Refreshed and rescued blocks, the
cold-block ranking and block maxima, keys scored, the final top-k set, every
policy-state array and every metric of the reference's metrics dict must
match exactly.  The verifier scores themselves are checked against float64
closed forms (head path: sum over the selected heads; dim path: the oracle's
sketch with float32-exact dot products) to 1e-5 of the score scale.

The sketch kernels (Hadamard rotation with per-stage rounding, dimension
selection, fake quantization, tensor scale) are compared bit for bit with
the oracle, which is pinned against Sylvester's matrix and torch's own
half-precision arithmetic.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsa_amd import approx, decode, verifier, verifier_scoring
from oracle import approx as A
from oracle import verifier as V
from oracle import verifier_scoring as S
from oracle.scores import relu_index_score

pytestmark = pytest.mark.gpu

TORCH_NAMES = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def trajectory(batch, length, steps, seed, rho=0.93):
    gen = torch.Generator().manual_seed(seed)
    q = [torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128)]
    for _ in range(steps):
        q.append(rho * q[-1] + math.sqrt(1 - rho * rho) * torch.randn(batch, 64, 128, generator=gen) / math.sqrt(128))
    w = torch.randn(batch, 64, generator=gen) / 8
    keys = torch.randn(batch, length + steps, 128, generator=gen)
    hot = torch.rand(batch, length + steps, generator=gen) < 0.01
    keys[hot] *= 4
    return [x.to(torch.bfloat16) for x in q], w, keys.to(torch.bfloat16)


def to_device_policy(policy: A.ApproxPolicy, gamma: float) -> approx.ApproxPolicy:
    fields = {f: getattr(policy, f) for f in approx.ApproxPolicy.__dataclass_fields__}
    fields["gamma"] = gamma
    return approx.ApproxPolicy(**fields)


# (name, path, width, block, rescue fraction, threshold in score sigmas or None,
#  temporal policy, wave, gamma in sigmas, sketch bits)
CASES = [
    ("head8_dynamic_b64", "head", 8, 64, 0.1, None, A.ApproxPolicy(name="static", cold_streak=0), 1, -2.0, None),
    ("head16_fixed_b32_thr", "head", 16, 32, 0.0, 0.5,
     A.ApproxPolicy(name="dyn", dynamic_threshold=True, order="previous_max", cold_streak=0), 4, -1.5, None),
    ("head40_b16", "head", 40, 16, 0.25, None,
     A.ApproxPolicy(name="ema", dynamic_threshold=True, order="bucket8", risk_model="ema", volatility_lambda=1.0,
                    cold_streak=0),
     8, -1.5, None),
    ("dim16_bf16_b64", "dim", 16, 64, 0.1, None, A.ApproxPolicy(name="static", cold_streak=0), 1, -2.0, None),
    ("dim32_int4_b64", "dim", 32, 64, 0.2, None,
     A.ApproxPolicy(name="dyn", dynamic_threshold=True, cold_streak=0), 2, -2.0, 4),
    ("dim16_int8_b128_thr", "dim", 16, 128, 0.0, 0.3, A.ApproxPolicy(name="static", cold_streak=0), 1, -2.5, 8),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_verifier_step_matches_oracle_trajectory(device, case) -> None:
    name, path, width, block, fraction, thr_sigma, policy, wave, gamma_sigma, bits = case
    batch, length, steps, k = 2, 4000, 5, 128
    print(f"verifier {name}", flush=True)
    qs, w, keys = trajectory(batch, length, steps, seed=width * 7 + block)
    w, keys = w.to(device), keys.to(device)
    _, scores0 = decode.indexer_topk(qs[0].to(device), w, keys[:, :length].contiguous(), k, return_scores=True)
    sigma = float(scores0.std())
    gamma = gamma_sigma * sigma
    threshold = None if thr_sigma is None else float(np.float32(thr_sigma * sigma * 0.5))
    ratio = width / 64 if path == "head" else width / 128
    cfg = dict(name=name, path=path, width=width, score_ratio=ratio, block_size=block, rescue_fraction=fraction,
               sketch_bytes_per_token=0.0 if path == "head" else width * (bits or 16) / 8)
    gpu_cfg = verifier.VerifierConfig(**cfg)
    cpu_cfg = V.VerifierConfig(**cfg)
    gpu_policy = to_device_policy(policy, gamma)
    cpu_policy = policy.with_gamma(gamma)
    state = approx.initialize_state(scores0, k=k, block_size=block, capacity=length + steps)
    host0 = scores0.cpu().numpy()
    oracle = [A.initialize_state(host0[b], k=k, block_size=block) for b in range(batch)]

    dims = np.linspace(0, 127, width).astype(np.int64) if width == 16 else np.sort(
        np.random.default_rng(1582).choice(128, width, replace=False))
    key_sketch = key_scale = query_scale = None
    if path == "dim":
        key_vals = S.normalized_hadamard(keys.float().cpu().numpy(), "bf16")[..., dims]
        if bits is not None:
            key_scale = S.quantize_scale(key_vals, bits)
            query_scale = 0.5 * key_scale
        key_sketch = verifier.sketch_keys(keys, dims, bits=bits, scale=key_scale)
    fixed_ids = torch.arange(0, 64, 64 // width if 64 % width == 0 else 1, device=device)[:width].to(torch.int32)

    rescued_total = 0
    cold_total = 0
    for t in range(1, steps + 1):
        cur = length + t
        q = qs[t].to(device)
        dense = decode.indexer_topk(q, w, keys[:, :cur].contiguous(), k, return_scores=True)[1]
        kwargs = {}
        if path == "head":
            ids = verifier_scoring.dynamic_head_indices(w, width, "high_weight") if width != 16 else fixed_ids
            kwargs["head_ids"] = ids
        else:
            kwargs["query_sketch"] = verifier.sketch_queries(q, dims, bits=bits, scale=query_scale)
            kwargs["key_sketch"] = key_sketch
            kwargs["sketch_scale"] = key_scale
        got = verifier.verifier_step(state, q, w, keys[:, :cur], policy=gpu_policy, config=gpu_cfg, step=t,
                                     wave=wave, promotion_threshold=threshold, **kwargs)
        dense_h = dense.cpu().numpy()
        vs = got.verifier_scores.cpu().numpy()
        host = {f: getattr(got, f).cpu().numpy() for f in
                ("topk", "scores", "block_scores", "cold_count", "evaluated_blocks", "rescued_blocks", "ranking",
                 "qk_scored", "counts")}
        st = state.host()
        for b in range(batch):
            where = f"{name} step {t} row {b}"
            oracle[b], metrics, details = V.verifier_step(
                oracle[b], dense_h[b], vs[b], policy=cpu_policy, config=cpu_cfg, k=k, step=t,
                previous_length=cur - 1, promotion_threshold=threshold, wave=wave,
            )
            cold = np.zeros(cur, dtype=bool)
            cold[details["cold"]] = True
            np.testing.assert_array_equal(np.isfinite(vs[b]), cold, err_msg=f"{where}: cold keys")
            nb = host["block_scores"].shape[1]
            cold_blocks = np.zeros(nb, dtype=bool)
            cold_blocks[np.unique(details["cold"] // block)] = True
            np.testing.assert_array_equal(host["cold_count"][b] > 0, cold_blocks, err_msg=f"{where}: cold blocks")
            np.testing.assert_array_equal(host["block_scores"][b][cold_blocks], details["block_scores"][cold_blocks],
                                          err_msg=f"{where}: block scores")
            ranking = host["ranking"][b]
            np.testing.assert_array_equal(ranking[ranking >= 0], details["block_ranking"], err_msg=f"{where}: ranking")
            rescued = np.zeros(nb, dtype=bool)
            rescued[details["rescued_blocks"]] = True
            np.testing.assert_array_equal(host["rescued_blocks"][b], rescued, err_msg=f"{where}: rescued")
            assert sorted(host["topk"][b].tolist()) == sorted(details["approximate"].tolist()), where
            exact = details["exact_candidates"]
            np.testing.assert_array_equal(np.flatnonzero(np.isfinite(host["scores"][b])), exact, err_msg=where)
            np.testing.assert_array_equal(host["scores"][b][exact], dense_h[b][exact], err_msg=where)
            assert int(host["qk_scored"][b]) == metrics["temporal_exact_tokens"], where
            assert host["counts"][b].tolist() == [
                metrics["cold_tokens_scanned"], metrics["cold_blocks_scanned"], metrics["rescue_blocks"],
                metrics["rescue_exact_tokens"]], where
            for field in ("last_max", "ema", "volatility", "age", "cold_streak"):
                np.testing.assert_array_equal(st[field][b], getattr(oracle[b], field), err_msg=f"{where}: {field}")
            mine = verifier.verifier_metrics(got, dense, config=gpu_cfg, policy=gpu_policy, step=t, row=b,
                                             promotion_threshold=threshold)
            assert set(mine) == set(metrics)
            for field, want in metrics.items():
                have = mine[field]
                if isinstance(want, float) and math.isnan(want):
                    assert math.isnan(have), (where, field)
                else:
                    assert have == want, (where, field, have, want)
            rescued_total += int(rescued.sum())
            # the verifier scores themselves, against float64 closed forms
            qh = q[b].float().cpu().numpy()
            wh = w[b].float().cpu().numpy()
            kh = keys[b, :cur].float().cpu().numpy()
            ck = np.flatnonzero(cold)[:600]
            cold_total += ck.size
            if ck.size == 0:
                continue
            if path == "head":
                ids_b = kwargs["head_ids"].cpu().numpy()
                ids_b = ids_b[b] if ids_b.ndim == 2 else ids_b
                want_v = relu_index_score(qh[ids_b], kh[ck], wh[ids_b])
            else:
                q_s = kwargs["query_sketch"][b].float().cpu().numpy()
                if bits is None:
                    k_s = key_sketch[b, ck].float().cpu().numpy()
                else:
                    k_s = S.round_bf16(key_sketch[b, ck].cpu().numpy().astype(np.float32) * np.float32(key_scale))
                want_v = relu_index_score(q_s, k_s, wh)
            scale = float(np.abs(want_v).max()) + 1e-6
            np.testing.assert_allclose(vs[b][ck], want_v, rtol=0, atol=1e-5 * scale, err_msg=f"{where}: verifier scores")
    assert cold_total > 0, "no cold keys: the case does not exercise the verifier"
    if fraction > 0 or threshold is not None:
        assert rescued_total > 0, "nothing was rescued: the case does not exercise the rescue"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("dim", [8, 128])
def test_hadamard_matches_oracle_bit_for_bit(device, dtype, dim) -> None:
    gen = torch.Generator().manual_seed(dim)
    x = (torch.randn(37, 3, dim, generator=gen) * 2).to(dtype)
    got = verifier_scoring.normalized_hadamard(x.to(device)).float().cpu().numpy()
    want = S.normalized_hadamard(x.float().numpy(), TORCH_NAMES[dtype])
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_sketch_quantization_matches_oracle(device, bits) -> None:
    gen = torch.Generator().manual_seed(bits)
    x = (torch.randn(300, 128, generator=gen) * 3).to(torch.bfloat16)
    dims = np.array([0, 3, 17, 31, 32, 63, 64, 65, 90, 101, 120, 127, 5, 6, 7, 8])
    vals = S.normalized_hadamard(x.float().numpy(), "bf16")[:, dims]
    want_v, scale, want_c = S.fake_symmetric_quantize(vals, bits, dtype="bf16")
    xd = x.to(device)
    got_c = verifier.dim_sketch(xd, dims, bits=bits, scale=scale, codes=True).cpu().numpy()
    got_v = verifier.dim_sketch(xd, dims, bits=bits, scale=scale).float().cpu().numpy()
    np.testing.assert_array_equal(got_c, want_c)
    np.testing.assert_array_equal(got_v, want_v)
    # tensor scale computed on the device (max |v| / limit, one host sync)
    auto = verifier.dim_sketch(xd, dims, bits=bits).float().cpu().numpy()
    np.testing.assert_array_equal(auto, want_v)
    fq, fscale = verifier_scoring.fake_symmetric_quantize(torch.from_numpy(vals).to(torch.bfloat16).to(device), bits)
    assert fscale == scale
    np.testing.assert_array_equal(fq.float().cpu().numpy(), want_v)


@pytest.mark.parametrize("rotation,bits", [("none", None), ("hadamard", None), ("hadamard", 4)])
def test_score_dim_sparse_matches_oracle(device, rotation, bits) -> None:
    gen = torch.Generator().manual_seed(11)
    q = (torch.randn(3, 64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16)
    k = torch.randn(1000, 128, generator=gen).to(torch.bfloat16)
    w = torch.randn(3, 64, generator=gen) / 8
    dims = np.sort(np.random.default_rng(5).choice(128, 32, replace=False))
    got = verifier_scoring.score_dim_sparse(q.to(device), w.to(device), k.to(device), dims, rotation=rotation,
                                            bits=bits).cpu().numpy()
    want = S.score_dim_sparse(q.float().numpy(), w.numpy(), k.float().numpy(), dims, rotation=rotation, bits=bits,
                              dtype="bf16", round_dots=False)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5 * float(np.abs(want).max()))


def test_full_width_dim_path_equals_head_path(device) -> None:
    # the reference's own identity (tests/test_verifier_scoring.py:25-32) on the GPU kernels
    gen = torch.Generator().manual_seed(1582)
    q = torch.randn(3, 4, 128, generator=gen).to(torch.bfloat16).to(device)
    k = torch.randn(200, 128, generator=gen).to(torch.bfloat16).to(device)
    w = torch.randn(3, 4, generator=gen).to(device)
    head = verifier_scoring.score_head_sparse(q, w, k, torch.arange(4)).cpu().numpy()
    dim = verifier_scoring.score_dim_sparse(q, w, k, torch.arange(128)).cpu().numpy()
    np.testing.assert_allclose(head, dim, rtol=0, atol=1e-5 * float(np.abs(head).max()))


def test_verifier_step_rejects_bad_inputs(device) -> None:
    scores = torch.randn(1, 512, device=device)
    state = approx.initialize_state(scores, k=16, block_size=64)
    q = torch.zeros(1, 64, 128, device=device, dtype=torch.bfloat16)
    w = torch.zeros(1, 64, device=device)
    keys = torch.zeros(1, 512, 128, device=device, dtype=torch.bfloat16)
    cfg = verifier.VerifierConfig(name="h", path="head", width=8, score_ratio=0.125, block_size=64)
    pol = approx.ApproxPolicy("s")
    with pytest.raises(ValueError, match="head_ids"):
        verifier.verifier_step(state, q, w, keys, policy=pol, config=cfg, step=1)
    with pytest.raises(ValueError, match="block_size"):
        verifier.verifier_step(state, q, w, keys, policy=pol, step=1, head_ids=torch.arange(8, device=device),
                               config=verifier.VerifierConfig(name="h", path="head", width=8, score_ratio=0.1,
                                                              block_size=32))
    dim_cfg = verifier.VerifierConfig(name="d", path="dim", width=12, score_ratio=0.1, block_size=64)
    with pytest.raises(ValueError, match="sketch"):
        verifier.verifier_step(state, q, w, keys, policy=pol, config=dim_cfg, step=1)
