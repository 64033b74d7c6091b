"""GPU parity of the sidecar encoder epilogues (RoPE, key LayerNorm + RoPE +
cache append, query RoPE + head-weight scale) against the oracle
(oracle/sidecar.py, reference sidecar.py:10-88), fed the same projections.

The angle of pair i is position * theta^(-i/half) in fp32 on both sides; a
one-ulp difference between the device's and the host's powf moves it by
position * 2^-24 radians, so the tolerance grows with the position.  In
bf16 a rounding boundary can move one result by one bf16 ulp.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsa_amd import _lib, sidecar
from oracle import sidecar as O

pytestmark = pytest.mark.gpu


def _tol(x: np.ndarray, pos: np.ndarray, bf16: bool, extra_dims: int = 1) -> np.ndarray:
    mag = np.abs(x).max(axis=-1, keepdims=True)
    p = pos.reshape(pos.shape + (1,) * extra_dims).astype(np.float64)
    angle = (p + 1) * 2.0**-22
    ulp = 2.0**-7 if bf16 else 2.0**-21
    return mag * (angle + ulp) * 2 + 1e-7


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("tokens,heads,dim,max_pos", [(37, 64, 128, 4096), (5, 4, 8, 20), (16, 1, 128, 100_000)])
def test_rope_matches_oracle(device, dtype, tokens, heads, dim, max_pos) -> None:
    print(f"rope {dtype} tokens={tokens} heads={heads} dim={dim} max_pos={max_pos}", flush=True)
    gen = torch.Generator().manual_seed(tokens * 7 + dim)
    x = torch.randn(tokens, heads, dim, generator=gen).to(dtype)
    pos = torch.randint(0, max_pos, (tokens,), generator=gen)
    got = sidecar.apply_noninterleaved_rope(x.to(device), pos.to(device)).float().cpu().numpy()
    bf16 = dtype == torch.bfloat16
    want = O.apply_noninterleaved_rope(x.float().numpy(), pos.numpy(), bf16=bf16)
    diff = np.abs(got - want)
    assert np.all(diff <= _tol(want, pos.numpy(), bf16, 2)), float(diff.max())
    if bf16:
        # bf16 rounding hides the fp32 ulp differences of cos / sin / pow:
        # almost every element is identical
        assert np.mean(diff == 0) > (0.99 if max_pos <= 4096 else 0.5)
        np.testing.assert_array_equal(O.round_bf16(got), got)


def test_rope_position_zero_is_identity(device) -> None:
    x = torch.randn(3, 64, 128, device=device)
    out = sidecar.apply_noninterleaved_rope(x, torch.zeros(3, dtype=torch.int64, device=device))
    assert torch.equal(out, x)


@pytest.mark.parametrize("proj_dtype,out_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                                  (torch.float32, torch.bfloat16)])
def test_key_epilogue_appends_into_cache(device, proj_dtype, out_dtype) -> None:
    print(f"key epilogue {proj_dtype} -> {out_dtype}", flush=True)
    gen = torch.Generator().manual_seed(11)
    tokens, dim, cache_rows = 24, 128, 300
    proj = (torch.randn(tokens, dim, generator=gen) * 2 + 0.5).to(proj_dtype)
    ln_w = torch.randn(dim, generator=gen)
    ln_b = torch.randn(dim, generator=gen)
    pos = torch.randint(0, 4096, (tokens,), generator=gen)
    rows = torch.randperm(cache_rows, generator=gen)[:tokens]
    cache = torch.full((cache_rows, dim), -7.0, dtype=out_dtype)
    # device copies held for the duration of the asynchronous launch
    cache_d, proj_d, ln_w_d, ln_b_d, pos_d, rows_d = (t.to(device) for t in (cache, proj, ln_w, ln_b, pos, rows))
    _lib.call(
        "dsa_encode_keys_epilogue", _lib.ptr(proj_d), _lib.dtype_code(proj_dtype), dim,
        _lib.ptr(ln_w_d), _lib.ptr(ln_b_d), 1e-6, _lib.ptr(pos_d), 64, 10_000.0,
        _lib.ptr(cache_d), _lib.dtype_code(out_dtype), dim, _lib.ptr(rows_d), cache_rows, tokens, dim,
        torch.cuda.current_stream().cuda_stream,
    )
    got = cache_d.float().cpu().numpy()
    bf16 = out_dtype == torch.bfloat16
    want = O.encode_keys_epilogue(proj.float().numpy(), ln_w.numpy(), ln_b.numpy(), pos.numpy(), 64, bf16=bf16)
    r = rows.numpy()
    diff = np.abs(got[r] - want)
    # LayerNorm's fp32 sums run in a different order on the two sides
    tol = _tol(want, pos.numpy(), bf16, 1) + np.abs(want) * (2.0**-7 if bf16 else 4e-6)
    assert np.all(diff <= tol), float(diff.max())
    untouched = np.ones(cache_rows, dtype=bool)
    untouched[r] = False
    assert np.all(got[untouched] == -7.0)


def test_query_epilogue(device) -> None:
    gen = torch.Generator().manual_seed(12)
    tokens = 16
    proj = torch.randn(tokens, 64, 128, generator=gen).to(torch.bfloat16)
    proj_w = torch.randn(tokens, 64, generator=gen)
    pos = torch.randint(0, 32768, (tokens,), generator=gen)
    q = torch.empty(tokens, 64, 128, dtype=torch.bfloat16, device=device)
    w = torch.empty(tokens, 64, device=device)
    proj_d, proj_w_d, pos_d = proj.to(device), proj_w.to(device), pos.to(device)
    _lib.call(
        "dsa_encode_queries_epilogue", _lib.ptr(proj_d), _lib.ptr(proj_w_d), _lib.ptr(pos_d),
        64, 10_000.0, float((64 * 128) ** -0.5), _lib.ptr(q), _lib.ptr(w), tokens, 64, 128, _lib.DTYPE_BF16,
        torch.cuda.current_stream().cuda_stream,
    )
    want_q, want_w = O.encode_queries_epilogue(proj.float().numpy(), proj_w.numpy(), pos.numpy(), 64, bf16=True)
    got = q.float().cpu().numpy()
    assert np.all(np.abs(got - want_q) <= _tol(want_q, pos.numpy(), True, 2))
    np.testing.assert_array_equal(w.cpu().numpy(), want_w)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_encoders_match_oracle(device, dtype) -> None:
    """LightningIndexerSidecar's encoders (18 tokens: the projection GEMM,
    with the query RoPE fused in bf16) against the oracle: its float64
    projections (the kernel's may differ by one bf16 rounding, or by fp32
    accumulation order) through its epilogues."""

    torch.manual_seed(13)
    module = sidecar.LightningIndexerSidecar(hidden_size=512).to(device=device, dtype=dtype)
    with torch.no_grad():
        module.k_norm.weight.normal_()
        module.k_norm.bias.normal_()
    hidden = torch.randn(2, 9, 512, device=device, dtype=dtype)
    pos = torch.arange(9, device=device).repeat(2, 1) + 1000
    with torch.no_grad():
        keys = module.encode_keys(hidden, pos)
        queries, weights = module.encode_queries(hidden, pos)
    bf16 = dtype == torch.bfloat16
    h = hidden.float().cpu().numpy()
    proj_k = O.project(h, module.wk.weight.detach().float().cpu().numpy(), bf16=bf16)
    proj_q = O.project(h, module.wq.weight.detach().float().cpu().numpy(), bf16=bf16).reshape(2, 9, 64, 128)
    proj_w = O.project(h, module.weights_proj.weight.detach().float().cpu().numpy())
    p = pos.cpu().numpy()
    want_k = O.encode_keys_epilogue(proj_k, module.k_norm.weight.detach().float().cpu().numpy(),
                                    module.k_norm.bias.detach().float().cpu().numpy(), p, 64, bf16=bf16)
    want_q, want_w = O.encode_queries_epilogue(proj_q, proj_w, p, 64, bf16=bf16)
    got_k = keys.float().cpu().numpy()
    tol_k = _tol(want_k, p, bf16, 1) + np.abs(want_k) * (2.0**-7 if bf16 else 4e-6)
    assert np.all(np.abs(got_k - want_k) <= tol_k)
    assert np.all(np.abs(queries.float().cpu().numpy() - want_q) <= _tol(want_q, p, bf16, 2))
    np.testing.assert_allclose(weights.cpu().numpy(), want_w, rtol=1e-5, atol=1e-6 * np.abs(want_w).max())


def test_reference_toy_shapes(device) -> None:
    """The reference test's configuration (tests/test_sidecar.py:10-19):
    hidden 16, 4 heads of 8 dims, rope_dim 4."""

    torch.manual_seed(1)
    module = sidecar.LightningIndexerSidecar(hidden_size=16, heads=4, head_dim=8, rope_dim=4).to(device)
    query = torch.randn(2, 3, 16, device=device)
    keys = torch.randn(2, 7, 16, device=device)
    q_pos = torch.arange(3, device=device).repeat(2, 1)
    k_pos = torch.arange(7, device=device).repeat(2, 1)
    with torch.no_grad():
        enc_k = module.encode_keys(keys, k_pos)
        enc_q, w = module.encode_queries(query, q_pos)
    assert enc_k.shape == (2, 7, 8) and enc_q.shape == (2, 3, 4, 8) and w.shape == (2, 3, 4)
    proj = torch.nn.functional.linear(keys, module.wk.weight).detach().cpu().numpy()
    want = O.encode_keys_epilogue(proj, module.k_norm.weight.detach().cpu().numpy(),
                                  module.k_norm.bias.detach().cpu().numpy(), k_pos.cpu().numpy(), 4)
    np.testing.assert_allclose(enc_k.cpu().numpy(), want, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError, match="64 heads x 128 dims"):
        module(query, keys, q_pos, k_pos)


def test_module_appends_keys_into_cache(device) -> None:
    torch.manual_seed(14)
    module = sidecar.LightningIndexerSidecar(hidden_size=256).to(device=device, dtype=torch.bfloat16)
    cache = torch.zeros(64, 128, device=device, dtype=torch.bfloat16)
    hidden = torch.randn(4, 256, device=device, dtype=torch.bfloat16)
    pos = torch.tensor([10, 11, 12, 13], device=device)
    rows = torch.tensor([3, 40, 7, 63], device=device)
    with torch.no_grad():
        module.encode_keys(hidden, pos, out=cache, out_rows=rows)
        direct = module.encode_keys(hidden, pos)
    assert torch.equal(cache[rows], direct)
    rest = torch.ones(64, dtype=torch.bool, device=device)
    rest[rows] = False
    assert torch.count_nonzero(cache[rest]) == 0
    # rows outside the cache are skipped, the others still written
    cache.zero_()
    with torch.no_grad():
        module.encode_keys(hidden, pos, out=cache, out_rows=torch.tensor([5, 64, -1, 9], device=device))
    assert torch.equal(cache[5], direct[0]) and torch.equal(cache[9], direct[3])
    assert torch.count_nonzero(cache) == torch.count_nonzero(direct[0]) + torch.count_nonzero(direct[3])


def test_forward_scores_match_float64(device) -> None:
    """Encoders then the HIP scoring kernel at 64 x 128 in bf16 against the
    float64 score of the oracle's encoded rows (bf16 tolerance)."""

    torch.manual_seed(15)
    module = sidecar.LightningIndexerSidecar(hidden_size=512).to(device=device, dtype=torch.bfloat16)
    qh = torch.randn(2, 1, 512, device=device, dtype=torch.bfloat16)
    kh = torch.randn(2, 300, 512, device=device, dtype=torch.bfloat16)
    qp = torch.full((2, 1), 299, device=device)
    kp = torch.arange(300, device=device).repeat(2, 1)
    with torch.no_grad():
        scores = module(qh, kh, qp, kp).float().cpu().numpy()
        q, w = module.encode_queries(qh, qp)
        k = module.encode_keys(kh, kp)
    qn = q.float().cpu().numpy().astype(np.float64)
    kn = k.float().cpu().numpy().astype(np.float64)
    wn = w.cpu().numpy().astype(np.float64)
    dots = np.einsum("bqhd,bkd->bqhk", qn, kn)
    want = (np.maximum(dots, 0) * wn[..., None]).sum(axis=2)
    scale = (np.abs(dots) * np.abs(wn)[..., None]).sum(axis=2)
    assert np.all(np.abs(scores - want) <= 1e-5 * scale + 1e-6)


@pytest.mark.parametrize("tokens", [1, 5, 16])
def test_decode_projection_kernel_matches_float64(device, tokens) -> None:
    """dsa_project_rows (the decode-step projections): bf16 outputs within one
    bf16 rounding of the float64 product, fp32 weights_proj to 1e-5 (larger
    batches run dsa_project_gemm, tested in test_gpu_sidecar_gemm.py)."""

    torch.manual_seed(tokens)
    module = sidecar.LightningIndexerSidecar(hidden_size=2048).to(device=device, dtype=torch.bfloat16).eval()
    hidden = torch.randn(tokens, 2048, device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        q = module._project(hidden, module.wq.weight).float().cpu().numpy().astype(np.float64)
        k = module._project(hidden, module.wk.weight).float().cpu().numpy().astype(np.float64)
        w = module._project(hidden, module.weights_proj.weight, fp32=True).cpu().numpy().astype(np.float64)
    h64 = hidden.float().cpu().numpy().astype(np.float64)
    for got, weight in ((q, module.wq.weight), (k, module.wk.weight)):
        want = h64 @ weight.detach().float().cpu().numpy().astype(np.float64).T
        # one bf16 rounding of the exact product (plus fp32 accumulation error)
        np.testing.assert_allclose(got, want, rtol=2 ** -8, atol=1e-4 * np.abs(want).max())
    want_w = h64 @ module.weights_proj.weight.detach().float().cpu().numpy().astype(np.float64).T
    np.testing.assert_allclose(w, want_w, rtol=1e-5, atol=1e-6 * np.abs(want_w).max())


@pytest.mark.gpu
@pytest.mark.parametrize("tokens", [1, 5, 16])
def test_paired_projection_matches_separate_calls(device, tokens) -> None:
    """dsa_project_rows_pair (wq and weights_proj in one launch) gives the
    same bits as the two dsa_project_rows calls, and encode_queries takes it."""

    print(f"sidecar pair projection tokens={tokens}", flush=True)
    torch.manual_seed(100 + tokens)
    module = sidecar.LightningIndexerSidecar(hidden_size=2048).to(device=device, dtype=torch.bfloat16).eval()
    module.weights_proj.to(torch.float32)
    hidden = torch.randn(tokens, 2048, device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        pair = module._project_pair(hidden, module.wq.weight, module.weights_proj.weight)
        assert pair is not None
        q = module._project(hidden, module.wq.weight)
        w = module._project(hidden, module.weights_proj.weight, fp32=True)
    assert torch.equal(pair[0].view(torch.int16), q.view(torch.int16))
    assert torch.equal(pair[1].view(torch.int32), w.view(torch.int32))
