"""GPU parity of the sidecar's projection GEMM (dsa_project_gemm: wq / wk /
weights_proj of reference sidecar.py:55-58 for batches above a decode step)
against the oracle (oracle/sidecar.py), up to the C4 token count (4096).

bf16 projections: the kernel accumulates in fp32 and rounds once, the oracle
sums in float64 and rounds via float32; the two can differ by one bf16 ulp
where the exact sum lies within the fp32 accumulation error of a rounding
boundary.  fp32 projections: within 1e-5 relative of the float64 sum.  The
fused query RoPE is compared bit for bit with the unfused GEMM followed by
the HIP query epilogue (same cos / sin, same per-op rounding), and against
the oracle's epilogue within the angle tolerance of the epilogue tests.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from dsa_amd import _lib, sidecar
from oracle import sidecar as O

pytestmark = pytest.mark.gpu


def _bf16_ulp(x: np.ndarray) -> np.ndarray:
    """One bf16 ulp at |x| (the spacing of bf16 values there)."""

    mag = np.maximum(np.abs(x), np.float32(2.0**-126)).astype(np.float32)
    return np.exp2(np.floor(np.log2(mag)) - 7)


def _module(hidden_size=2048, dtype=torch.bfloat16, seed=0, device="cuda"):
    torch.manual_seed(seed)
    m = sidecar.LightningIndexerSidecar(hidden_size=hidden_size).to(device=device, dtype=dtype).eval()
    m.weights_proj.to(torch.float32)
    return m


@pytest.mark.parametrize("tokens", [17, 300, 4096, 4099])
def test_bf16_projections_match_float64(device, tokens) -> None:
    print(f"gemm bf16 projections tokens={tokens}", flush=True)
    m = _module(seed=tokens, device=device)
    hidden = torch.randn(tokens, 2048, device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        q = m._project(hidden, m.wq.weight).float().cpu().numpy()
        k = m._project(hidden, m.wk.weight).float().cpu().numpy()
    h = hidden.float().cpu().numpy()
    for got, weight in ((q, m.wq.weight), (k, m.wk.weight)):
        wn = weight.detach().float().cpu().numpy()
        want = O.project(h, wn, bf16=True)
        # One bf16 ulp, plus the fp32 accumulation error of the k-sum, which
        # decides the rounding where the sum cancels to near zero: at most
        # 2^-20 of the sum of |products| (the kernel's measured error is about
        # 2^-28 of it; torch's GEMM gives the same outputs there).
        acc = 2.0**-20 * (np.abs(h).astype(np.float64) @ np.abs(wn).astype(np.float64).T)
        diff = np.abs(got - want)
        assert np.all(diff <= _bf16_ulp(want) + acc), float((diff - _bf16_ulp(want) - acc).max())
        np.testing.assert_array_equal(O.round_bf16(got), got)  # the outputs are bf16 values
        assert np.mean(diff == 0) > 0.99


@pytest.mark.parametrize("tokens,hidden_f32", [(17, False), (4096, False), (1000, True)])
def test_fp32_projection_and_scale(device, tokens, hidden_f32) -> None:
    # weights_proj on hidden.float() (bf16 hidden widened exactly, or fp32),
    # and the head-weight scale as one fp32 product.
    print(f"gemm fp32 projection tokens={tokens} hidden_f32={hidden_f32}", flush=True)
    m = _module(seed=7 + tokens, device=device)
    hidden = torch.randn(tokens, 2048, device=device, dtype=torch.float32 if hidden_f32 else torch.bfloat16)
    scale = float((64 * 128) ** -0.5)
    with torch.no_grad():
        plain = m._project(hidden, m.weights_proj.weight, fp32=True).cpu().numpy()
        scaled = m._project(hidden, m.weights_proj.weight, fp32=True, scale=scale).cpu().numpy()
    want = O.project(hidden.float().cpu().numpy(), m.weights_proj.weight.detach().cpu().numpy())
    np.testing.assert_allclose(plain, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
    np.testing.assert_array_equal(scaled, (plain * np.float32(scale)).astype(np.float32))


@pytest.mark.parametrize("tokens", [17, 4096])
def test_fused_query_rope_matches_epilogue(device, tokens) -> None:
    # encode_queries above a decode step: the RoPE in the wq GEMM's output
    # stage equals the plain GEMM + the HIP query epilogue bit for bit, and the
    # oracle's epilogue fed that GEMM's projection within the angle tolerance.
    print(f"gemm fused query rope tokens={tokens}", flush=True)
    m = _module(seed=100 + tokens, device=device)
    hidden = torch.randn(2, tokens, 2048, device=device, dtype=torch.bfloat16)
    pos = (torch.arange(tokens, device=device) + 123).repeat(2, 1)
    with torch.no_grad():
        queries, weights = m.encode_queries(hidden, pos)
        proj = m._project(hidden, m.wq.weight)
        proj_w = m._project(hidden, m.weights_proj.weight, fp32=True)
    flat = proj.reshape(2 * tokens, 64 * 128).contiguous()
    want_q = torch.empty_like(flat)
    want_w = torch.empty(2 * tokens, 64, device=device)
    p = pos.reshape(-1).contiguous()
    _lib.call("dsa_encode_queries_epilogue", flat.data_ptr(), proj_w.reshape(-1, 64).contiguous().data_ptr(),
              p.data_ptr(), 64, float(m.rope_theta), float((64 * 128) ** -0.5), want_q.data_ptr(), want_w.data_ptr(),
              2 * tokens, 64, 128, _lib.DTYPE_BF16, _lib.stream_of(flat))
    assert queries.shape == (2, tokens, 64, 128) and weights.shape == (2, tokens, 64)
    assert torch.equal(queries.reshape(2 * tokens, -1).view(torch.int16), want_q.view(torch.int16))
    assert torch.equal(weights.reshape(2 * tokens, -1).view(torch.int32), want_w.view(torch.int32))
    # The oracle's epilogue on the same projection (rows of 4096 tokens: check 2 x 64 of them).
    rows = np.r_[0:64, tokens - 64:tokens] if tokens > 128 else np.arange(tokens)
    pr = proj[0, rows].float().cpu().numpy().reshape(len(rows), 64, 128)
    pw = proj_w[0, rows].cpu().numpy()
    oq, ow = O.encode_queries_epilogue(pr, pw, pos[0, rows].cpu().numpy(), 64, bf16=True)
    got = queries[0, rows].float().cpu().numpy()
    mag = np.abs(oq).max(axis=-1, keepdims=True)
    angle = (pos[0, rows].cpu().numpy().astype(np.float64)[:, None, None] + 1) * 2.0**-22
    assert np.all(np.abs(got - oq) <= mag * (angle + 2.0**-7) * 2 + 1e-7)
    np.testing.assert_array_equal(weights[0, rows].cpu().numpy(), ow)


def test_fp32_module_and_small_shapes(device) -> None:
    # An fp32 module (hidden and weights fp32: the fp32 GEMM for every
    # projection) above a decode step, and the reference test's toy shape
    # (hidden 16, 4 heads of 8 dims: 8 key features) with 40 tokens.
    print("gemm fp32 module and toy shapes", flush=True)
    m = _module(hidden_size=512, dtype=torch.float32, seed=3, device=device)
    hidden = torch.randn(3, 50, 512, device=device)
    with torch.no_grad():
        q = m._project(hidden, m.wq.weight).cpu().numpy()
        k = m._project(hidden, m.wk.weight).cpu().numpy()
    h = hidden.cpu().numpy()
    for got, weight in ((q, m.wq.weight), (k, m.wk.weight)):
        want = O.project(h, weight.detach().cpu().numpy())
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
    torch.manual_seed(1)
    toy = sidecar.LightningIndexerSidecar(hidden_size=16, heads=4, head_dim=8, rope_dim=4).to(device)
    keys = torch.randn(2, 40, 16, device=device)
    k_pos = torch.arange(40, device=device).repeat(2, 1)
    with torch.no_grad():
        enc_k = toy.encode_keys(keys, k_pos)
    proj = O.project(keys.cpu().numpy(), toy.wk.weight.detach().cpu().numpy())
    want = O.encode_keys_epilogue(proj, toy.k_norm.weight.detach().cpu().numpy(),
                                  toy.k_norm.bias.detach().cpu().numpy(), k_pos.cpu().numpy(), 4)
    np.testing.assert_allclose(enc_k.cpu().numpy(), want, rtol=1e-4, atol=1e-4)


def test_strided_hidden_rows(device) -> None:
    # A hidden batch that is a column slice of a wider buffer (row stride >
    # width): the GEMM reads the rows in place.
    print("gemm strided hidden rows", flush=True)
    m = _module(seed=11, device=device)
    wide = torch.randn(300, 2048 + 64, device=device, dtype=torch.bfloat16)
    hidden = wide[:, :2048]
    with torch.no_grad():
        got = m._project(hidden, m.wk.weight)
        want = m._project(hidden.contiguous(), m.wk.weight)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
