"""Sidecar indexer: encoders and batched / multi-query scoring.

Reference: ``temporal_dsa/sidecar.py``.
  * ``apply_noninterleaved_rope`` (sidecar.py:10-28) and the encoders of
    ``LightningIndexerSidecar`` (sidecar.py:31-88): the projections wq / wk /
    weights_proj run in the library's own kernels, a weight-streaming kernel
    for a decode step (``dsa_project_rows``) and an MFMA GEMM for larger
    batches (``dsa_project_gemm``); the LayerNorm, RoPE, head-weight scaling
    and the key-cache append after them run in one HIP pass per row
    (``dsa_encode_keys_epilogue``, ``dsa_encode_queries_epilogue``,
    ``dsa_rope``), with torch's per-op rounding in the row dtype, or, for
    the queries of a bf16 batch, inside the GEMM's output stage.  The module
    runs in its parameter dtype (fp32 or bf16); autocast's mixed flow is not
    reproduced.
  * ``score_encoded`` (sidecar.py:89-107): ``[B,Q,H,D] x [B,K,D] -> [B,Q,K]``
    fp32, ``ReLU(q.k) * w`` summed over heads.

Differences of ``score_encoded`` from the reference, all documented at the call:
  * dots stay fp32 (the reference's bf16 einsum rounds each dot to bf16 before
    the ReLU; both agree within the 1e-2 relative bf16 tolerance);
  * ``causal=True`` masks key j of query t unless ``j <= t + causal_offset``
    (masked scores are -inf); the reference has no mask;
  * fp8 e4m3fn keys with one fp32 scale per 128 keys are accepted through
    ``key_scales`` ``[B, ceil(K/128)]``.
The KL loss and the teacher target (sidecar.py:123-137) belong to training
and are not part of this package.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from . import _lib
from .progressive_kernel import HEAD_DIM, HEADS

_ROW_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}


def score_encoded(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    *,
    key_chunk_size: int | None = None,
    causal: bool = False,
    causal_offset: int | None = None,
    key_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Indexer scores of every (query, key) pair, fp32 ``[B, Q, K]``.

    ``key_chunk_size`` is accepted for API compatibility; the kernel streams
    keys without materialising per-head dots, so no chunking is needed.
    ``causal_offset`` defaults to ``K - Q`` (the last query sees every key).
    """

    del key_chunk_size
    if queries.ndim != 4 or weights.shape != queries.shape[:-1]:
        raise ValueError("queries must be [batch,query,heads,dim]")
    if keys.ndim != 3 or keys.shape[0] != queries.shape[0]:
        raise ValueError("keys must be [batch,key,dim]")
    batch, num_queries, heads, dim = queries.shape
    length = keys.shape[1]
    if heads != HEADS or dim != HEAD_DIM or keys.shape[2] != HEAD_DIM:
        raise ValueError("expected 64 heads x 128 dims")
    if not (queries.is_cuda and weights.is_cuda and keys.is_cuda):
        raise ValueError("HIP kernels require GPU tensors")
    if queries.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("queries must be FP16/BF16")
    fp8 = keys.dtype == torch.float8_e4m3fn
    if fp8:
        if queries.dtype != torch.bfloat16:
            raise ValueError("fp8 keys are scored against BF16 queries")
        if key_scales is None or key_scales.shape != (batch, (length + 127) // 128):
            raise ValueError("fp8 keys need key_scales [batch, ceil(keys/128)]")
        key_scales = key_scales.to(device=keys.device, dtype=torch.float32).contiguous()
    elif keys.dtype != queries.dtype:
        raise ValueError("queries and keys must share FP16/BF16 dtype")
    if length == 0 or num_queries == 0 or batch == 0:
        return torch.empty((batch, num_queries, length), device=keys.device, dtype=torch.float32)
    queries = queries.contiguous()
    keys = keys.contiguous()
    weights = weights.to(torch.float32).contiguous()
    out = torch.empty((batch, num_queries, length), device=keys.device, dtype=torch.float32)
    offset = -1
    if causal:
        offset = length - num_queries if causal_offset is None else int(causal_offset)
        if offset < 0:
            raise ValueError("causal_offset must be non-negative")
    _lib.call(
        "dsa_score_queries",
        _lib.ptr(queries), HEADS * HEAD_DIM, _lib.ptr(weights), HEADS, None, 0, HEADS,
        _lib.ptr(keys), length, num_queries, _lib.ptr(key_scales), (length + 127) // 128,
        _lib.ptr(out), length, batch * num_queries, length, offset,
        _lib.dtype_code(keys.dtype), _lib.stream_of(keys),
    )
    return out


def score_encoded_topk(
    queries: torch.Tensor,
    weights: torch.Tensor,
    keys: torch.Tensor,
    k: int,
    *,
    causal: bool = False,
    causal_offset: int | None = None,
    return_values: bool = False,
):
    """``score_encoded`` (reference sidecar.py:89-107) and every query's exact
    top-k of its visible keys (``stable_topk``, metrics.py:9-22, in ascending
    index order) in one launch (``dsa_score_queries_topk``).

    Returns ``(scores [B, Q, K] fp32, indices [B, Q, k] int64)``, plus the
    selected values ``[B, Q, k]`` with ``return_values``.  A query with fewer
    than ``k`` visible keys returns all of them, padded with -1 (values -inf).
    Needs fp16/bf16 queries and keys, at least 4 queries per key set and at
    most 4096 keys.
    """

    if queries.ndim != 4 or weights.shape != queries.shape[:-1]:
        raise ValueError("queries must be [batch,query,heads,dim]")
    if keys.ndim != 3 or keys.shape[0] != queries.shape[0]:
        raise ValueError("keys must be [batch,key,dim]")
    batch, num_queries, heads, dim = queries.shape
    length = keys.shape[1]
    if heads != HEADS or dim != HEAD_DIM or keys.shape[2] != HEAD_DIM:
        raise ValueError("expected 64 heads x 128 dims")
    if not (queries.is_cuda and weights.is_cuda and keys.is_cuda):
        raise ValueError("HIP kernels require GPU tensors")
    if queries.dtype not in (torch.float16, torch.bfloat16) or keys.dtype != queries.dtype:
        raise ValueError("queries and keys must share FP16/BF16 dtype")
    if k <= 0:
        raise ValueError("k must be positive")
    if not 1 <= length <= 4096:
        raise ValueError("the fused top-k takes 1..4096 keys per key set")
    if num_queries < 4:
        raise ValueError("the fused top-k takes at least 4 queries per key set")
    offset = -1
    if causal:
        offset = length - num_queries if causal_offset is None else int(causal_offset)
        if offset < 0:
            raise ValueError("causal_offset must be non-negative")
    queries = queries.contiguous()
    keys = keys.contiguous()
    weights = weights.to(torch.float32).contiguous()
    scores = torch.empty((batch, num_queries, length), device=keys.device, dtype=torch.float32)
    indices = torch.empty((batch, num_queries, k), device=keys.device, dtype=torch.int64)
    values = torch.empty((batch, num_queries, k), device=keys.device, dtype=torch.float32) if return_values else None
    _lib.call(
        "dsa_score_queries_topk",
        _lib.ptr(queries), HEADS * HEAD_DIM, _lib.ptr(weights), HEADS, _lib.ptr(keys), length, num_queries,
        _lib.ptr(scores), length, batch * num_queries, length, offset, _lib.dtype_code(keys.dtype), int(k),
        _lib.ptr(indices), _lib.ptr(values), int(k), _lib.stream_of(keys),
    )
    if return_values:
        return scores, indices, values
    return scores, indices


def _row_dtype(t: torch.Tensor) -> int:
    try:
        return _ROW_DTYPES[t.dtype]
    except KeyError:
        raise ValueError("sidecar rows must be float32 or bfloat16") from None


def _token_positions(positions, shape, device) -> torch.Tensor:
    pos = torch.as_tensor(positions, device=device)
    if pos.shape != shape:
        pos = pos.expand(shape)
    return pos.to(torch.int64).contiguous().reshape(-1)


def apply_noninterleaved_rope(x: torch.Tensor, positions: torch.Tensor, *, theta: float = 10_000.0) -> torch.Tensor:
    """Non-interleaved RoPE (reference sidecar.py:10-28) of x ``[..., d]``;
    positions has shape ``x.shape[:-1]`` or ``x.shape[:-2]`` (one position
    per token, shared by its heads)."""

    if x.shape[-1] % 2:
        raise ValueError("RoPE dimension must be even")
    if not x.is_cuda:
        raise ValueError("HIP kernels require GPU tensors")
    dtype = _row_dtype(x)
    d = x.shape[-1]
    pos = torch.as_tensor(positions, device=x.device)
    if tuple(pos.shape) == tuple(x.shape[:-1]):
        heads = 1
        tokens_shape = x.shape[:-1]
    elif x.ndim >= 2 and tuple(pos.shape) == tuple(x.shape[:-2]):
        heads = x.shape[-2]
        tokens_shape = x.shape[:-2]
    else:
        raise ValueError("positions must match x.shape[:-1] or x.shape[:-2]")
    if d > 256:
        raise ValueError("RoPE rows of more than 256 dims are not supported")
    rows = x.contiguous()
    out = torch.empty_like(rows)
    tokens = math.prod(tokens_shape)
    _lib.call("dsa_rope", _lib.ptr(rows), _lib.ptr(out), _lib.ptr(_token_positions(pos, tokens_shape, x.device)),
              tokens, heads, d, d, float(theta), dtype, _lib.stream_of(rows))
    return out


class LightningIndexerSidecar(nn.Module):
    """The indexer sidecar (reference sidecar.py:31-121): same constructor,
    parameters and initialisation; the encoders' epilogues run in HIP."""

    def __init__(
        self,
        hidden_size: int = 2048,
        heads: int = 64,
        head_dim: int = 128,
        rope_dim: int = 64,
        rope_theta: float = 10_000.0,
    ) -> None:
        super().__init__()
        if not 0 <= rope_dim <= head_dim or rope_dim % 2:
            raise ValueError("rope_dim must be even and no larger than head_dim")
        self.hidden_size = hidden_size
        self.heads = heads
        self.head_dim = head_dim
        self.rope_dim = rope_dim
        self.rope_theta = rope_theta
        self.wq = nn.Linear(hidden_size, heads * head_dim, bias=False)
        self.wk = nn.Linear(hidden_size, head_dim, bias=False)
        self.k_norm = nn.LayerNorm(head_dim, eps=1e-6)
        self.weights_proj = nn.Linear(hidden_size, heads, bias=False, dtype=torch.float32)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        nn.init.normal_(self.wq.weight, mean=0.0, std=self.hidden_size**-0.5)
        nn.init.normal_(self.wk.weight, mean=0.0, std=self.hidden_size**-0.5)
        nn.init.normal_(self.weights_proj.weight, mean=0.0, std=self.hidden_size**-0.5)

    def _project(self, hidden: torch.Tensor, weight: torch.Tensor, *, fp32: bool = False,
                 scale: float | None = None, positions: torch.Tensor | None = None) -> torch.Tensor:
        """A Linear without bias (sidecar.py:55-58): ``hidden @ weight.T``, in
        the weight's dtype (bf16, or fp32 on ``hidden.float()`` with ``fp32``
        as weights_proj runs), times ``scale`` in fp32 when given.  A decode
        step (at most 16 bf16 tokens) streams the weights in
        ``dsa_project_rows``; larger batches, and fp32 modules, run the MFMA
        GEMM ``dsa_project_gemm``, which with ``positions`` also applies
        encode_queries' RoPE to every 128-dim head (bf16, rope_dim 64).
        Inference only: no autograd graph is kept."""

        kdim = hidden.shape[-1]
        if weight.ndim != 2 or weight.shape[1] != kdim:
            raise ValueError(f"hidden width {kdim} does not match the weight's {tuple(weight.shape)}")
        if not hidden.is_cuda or not weight.is_cuda:
            raise ValueError("HIP kernels require GPU tensors")
        tokens = hidden.numel() // kdim if kdim else 0
        features = weight.shape[0]
        w = weight.detach()
        if fp32 and w.dtype != torch.float32:
            w = w.float()
        if hidden.dtype not in (torch.bfloat16, torch.float32) or w.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("sidecar projections take bf16 or fp32 hidden states and weights")
        if w.dtype == torch.bfloat16 and hidden.dtype != torch.bfloat16:
            raise ValueError("a bf16 projection takes bf16 hidden states")
        w = w.contiguous()
        out_dtype = torch.float32 if w.dtype == torch.float32 else torch.bfloat16
        lead = hidden.shape[:-1]
        out = torch.empty((tokens, features), device=hidden.device, dtype=out_dtype)
        if tokens == 0:
            return out.reshape(*lead, features)
        flat = hidden.reshape(tokens, kdim)
        if flat.stride(-1) != 1 or flat.stride(0) % 8 or flat.data_ptr() % 16:
            flat = flat.contiguous()
        stream = _lib.stream_of(flat)
        decode = (tokens <= 16 and hidden.dtype == torch.bfloat16 and kdim % 32 == 0 and scale is None
                  and positions is None and (w.dtype == torch.float32 or features % 16 == 0))
        if decode:
            _lib.call("dsa_project_rows", _lib.ptr(flat), flat.stride(0), tokens, _lib.ptr(w),
                      _lib.DTYPE_F32 if w.dtype == torch.float32 else _lib.DTYPE_BF16, features, kdim, _lib.ptr(out),
                      features, stream)
            return out.reshape(*lead, features)
        if kdim % 8 or features % 4:
            raise ValueError("sidecar projections need a hidden width that is a multiple of 8 and a multiple of "
                             "4 output features")
        pos = None
        ws = None
        need = 0
        if positions is not None:
            pos = _token_positions(positions, lead, hidden.device)
            need = int(_lib.query("dsa_project_gemm_workspace_bytes", tokens))
            ws = _lib.workspace("rope_table", hidden.device, stream, need, zeroed=False)
        _lib.call("dsa_project_gemm", _lib.ptr(flat), _row_dtype(flat), flat.stride(0), tokens, kdim, _lib.ptr(w),
                  _row_dtype(w), features, _lib.ptr(out), features, float(1.0 if scale is None else scale),
                  _lib.ptr(pos), float(self.rope_theta), _lib.ptr(ws), need, stream)
        return out.reshape(*lead, features)

    def _project_pair(self, hidden: torch.Tensor, weight: torch.Tensor, weight_f32: torch.Tensor):
        """``(hidden @ weight.T, hidden.float() @ weight_f32.T)`` in one
        launch (``dsa_project_rows_pair``) for a decode step that fits the
        projection kernel, else ``None``; identical to two :meth:`_project`
        calls."""

        tokens = hidden.numel() // hidden.shape[-1] if hidden.shape[-1] else 0
        kdim = hidden.shape[-1]
        if not (hidden.is_cuda and 0 < tokens <= 16 and hidden.dtype == torch.bfloat16 and kdim % 32 == 0
                and weight.ndim == 2 and weight.shape[1] == kdim and weight_f32.ndim == 2 and weight_f32.shape[1] == kdim
                and weight.dtype == torch.bfloat16 and weight.shape[0] % 16 == 0 and weight_f32.dtype == torch.float32):
            return None
        flat = hidden.reshape(tokens, kdim)
        if flat.stride(-1) != 1 or flat.stride(0) % 8 or flat.data_ptr() % 16:
            flat = flat.contiguous()
        w = weight.detach().contiguous()
        wf = weight_f32.detach().contiguous()
        out = torch.empty((tokens, w.shape[0]), device=hidden.device, dtype=torch.bfloat16)
        out_f = torch.empty((tokens, wf.shape[0]), device=hidden.device, dtype=torch.float32)
        _lib.call("dsa_project_rows_pair", _lib.ptr(flat), flat.stride(0), tokens, kdim, _lib.ptr(w), w.shape[0],
                  _lib.ptr(out), w.shape[0], _lib.ptr(wf), wf.shape[0], _lib.ptr(out_f), wf.shape[0],
                  _lib.stream_of(flat))
        lead = hidden.shape[:-1]
        return out.reshape(*lead, w.shape[0]), out_f.reshape(*lead, wf.shape[0])

    def encode_keys(
        self,
        hidden: torch.Tensor,
        positions: torch.Tensor,
        *,
        out: torch.Tensor | None = None,
        out_rows: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """RoPE(LayerNorm(wk(hidden))) (sidecar.py:74-76) ``[..., head_dim]``.

        With ``out`` (a key cache ``[rows, head_dim]``, fp32 or bf16) and
        ``out_rows`` (int64, one cache row per token), the keys are written
        into the cache rows instead and ``out`` is returned: the decode step's
        append without a separate copy.  A token whose row lies outside the
        cache is not written.  Inference only: no autograd graph is kept.
        """

        if not hidden.is_cuda:
            raise ValueError("HIP kernels require GPU tensors")
        proj = self._project(hidden, self.wk.weight)
        tokens_shape = proj.shape[:-1]
        tokens = math.prod(tokens_shape)
        flat = proj.reshape(tokens, self.head_dim).contiguous()
        pos = _token_positions(positions, tokens_shape, hidden.device)
        ln_w = self.k_norm.weight.detach().to(torch.float32).contiguous()
        ln_b = self.k_norm.bias.detach().to(torch.float32).contiguous()
        if out is None:
            result = torch.empty_like(flat)
            rows = None
            target = result
        else:
            if out.ndim != 2 or out.shape[1] != self.head_dim or not out.is_contiguous():
                raise ValueError("out must be a contiguous [rows, head_dim] key cache")
            if out_rows is None or out_rows.numel() != tokens:
                raise ValueError("out_rows must give one cache row per token")
            # (rows outside the cache are skipped by the kernel: no host sync here)
            rows = out_rows.to(device=hidden.device, dtype=torch.int64).contiguous()
            target = out
        _lib.call(
            "dsa_encode_keys_epilogue", _lib.ptr(flat), _row_dtype(flat), self.head_dim, _lib.ptr(ln_w),
            _lib.ptr(ln_b), float(self.k_norm.eps), _lib.ptr(pos), self.rope_dim, float(self.rope_theta),
            _lib.ptr(target), _row_dtype(target), self.head_dim, _lib.ptr(rows), target.shape[0], tokens,
            self.head_dim, _lib.stream_of(flat),
        )
        if out is not None:
            return out
        return result.reshape(*tokens_shape, self.head_dim)

    def encode_queries(self, hidden: torch.Tensor, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(queries ``[..., heads, head_dim]``, weights ``[..., heads]`` fp32)
        (sidecar.py:78-88)."""

        if not hidden.is_cuda:
            raise ValueError("HIP kernels require GPU tensors")
        scale = float((self.heads * self.head_dim) ** -0.5)
        tokens = hidden.numel() // hidden.shape[-1] if hidden.shape[-1] else 0
        if (tokens > 16 and hidden.dtype == torch.bfloat16 and self.wq.weight.dtype == torch.bfloat16
                and self.head_dim == 128 and self.rope_dim == 64 and (self.heads * self.head_dim) % 256 == 0
                and hidden.shape[-1] % 8 == 0):
            # The RoPE of every head in the wq GEMM's output stage and the
            # head-weight scale in weights_proj's: no epilogue pass.
            lead = hidden.shape[:-1]
            queries = self._project(hidden, self.wq.weight, positions=positions)
            weights = self._project(hidden, self.weights_proj.weight, fp32=True, scale=scale)
            return queries.reshape(*lead, self.heads, self.head_dim), weights.reshape(*lead, self.heads)
        pair = self._project_pair(hidden, self.wq.weight, self.weights_proj.weight)
        if pair is None:
            proj = self._project(hidden, self.wq.weight)
            proj_w = self._project(hidden, self.weights_proj.weight, fp32=True)
        else:
            proj, proj_w = pair
        tokens_shape = proj.shape[:-1]
        tokens = math.prod(tokens_shape)
        flat = proj.reshape(tokens, self.heads * self.head_dim).contiguous()
        flat_w = proj_w.reshape(tokens, self.heads).contiguous()
        pos = _token_positions(positions, tokens_shape, hidden.device)
        queries = torch.empty_like(flat)
        weights = torch.empty_like(flat_w)
        _lib.call(
            "dsa_encode_queries_epilogue", _lib.ptr(flat), _lib.ptr(flat_w), _lib.ptr(pos), self.rope_dim,
            float(self.rope_theta), scale, _lib.ptr(queries),
            _lib.ptr(weights), tokens, self.heads, self.head_dim, _row_dtype(flat), _lib.stream_of(flat),
        )
        return (queries.reshape(*tokens_shape, self.heads, self.head_dim), weights.reshape(*tokens_shape, self.heads))

    def score_encoded(
        self,
        queries: torch.Tensor,
        weights: torch.Tensor,
        keys: torch.Tensor,
        *,
        key_chunk_size: int | None = None,
    ) -> torch.Tensor:
        """``[B,Q,H,D] x [B,K,D] -> [B,Q,K]`` (sidecar.py:89-107) on the HIP
        scoring kernel: 64 heads x 128 dims, bf16/fp16 queries (fp32 keys are
        cast to the query dtype, as autocast does in the reference's flow)."""

        if keys.is_floating_point() and keys.dtype == torch.float32 and queries.dtype != torch.float32:
            keys = keys.to(queries.dtype)
        return score_encoded(queries, weights, keys, key_chunk_size=key_chunk_size)

    def forward(
        self,
        query_hidden: torch.Tensor,
        key_hidden: torch.Tensor,
        query_positions: torch.Tensor,
        key_positions: torch.Tensor,
        *,
        key_chunk_size: int | None = None,
    ) -> torch.Tensor:
        queries, weights = self.encode_queries(query_hidden, query_positions)
        keys = self.encode_keys(key_hidden, key_positions)
        return self.score_encoded(queries, weights, keys, key_chunk_size=key_chunk_size)
