"""Per-workgroup phase timelines of the decode scoring kernel and of the fused
static temporal step, from the trace build of the library.

    python -m dsa_amd.build --trace
    python -m dsa_amd.phase_trace --config c2 [--out timeline.json]

The trace build (``-DDSA_PHASE_TRACE``) has thread 0 of every workgroup store
the GPU's 100 MHz wall clock at named points of the kernel.  Each run here is
queued behind a 512 MiB read, as the benchmark's cold-cache runs are; the log
of the last run is read back and every mark is reported relative to the
earliest workgroup start, as percentiles over workgroups and per XCD
(workgroups are dispatched to the 8 XCDs round-robin by blockIdx.x).

Configurations: ``c2`` (B=16, L=32768 bf16, K=2048 decode step), ``c5``
(B=4, L=131072 fp8, K=2048), ``c3-static`` (B=4, 16384 -> 16385 keys,
K=2048, block 64 static temporal step), ``c5-static`` (the same step on
C5's fp8 shape, 131071 -> 131072 keys, margin 0.25 sigma), ``c4-topk`` (the prefill top-512
of 4096 causal rows of 1..4096 scores; in this one the row-loaded mark waits
for the row, so the trace build's timing of that kernel differs slightly),
and ``c2-select`` / ``c5-select`` (the decode step's list select).

``c3-replay`` and ``c5-replay`` report instead, per row, the phase totals of
the dynamic temporal step's replay (temporal_resolve_kernel) over all of the
step's rounds: setup (kernel start to the group loop), the group loop and its
decisions, exact selects, joins and cut moves, the loop's steps, the listed
keys, and the tail after the loop (the running k largest written back with
its keys, or the step's top-k and keys scored; the -inf resets).  C3: block 16,
address order, 33-block groups, gamma = sigma of the score drift; C5: fp8,
block 64, previous-hot order, 96-block groups, gamma = 0.25 sigma.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .build import TRACE_LIBRARY

WALL_CLOCK_MHZ = 100.0
MARKS = {
    "dense": ["start", "first unit scored", "last unit scored", "list written"],
    "static": ["start", "seeds listed", "seeds scored", "threshold exchanged", "blocks decided", "units scored",
               "list written"],
    "topk": ["start", "row loaded", "range known", "cut located", "cut resolved", "slots scanned", "written"],
    "select": ["start", "entries counted, cut bin located", "cut resolved", "earlier lists counted", "written",
               "radix pass 0 counted", "radix pass 1 counted", "radix pass 2 counted"],
}
KERNEL_SYMBOL = {"dense": "dsa_trace_dense_scores", "static": "dsa_trace_temporal_static", "topk": "dsa_trace_topk",
                 "select": "dsa_trace_select_lists"}


def _c2(device):
    from . import decode

    gen = torch.Generator().manual_seed(1582)
    q = (torch.randn(16, 64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16).to(device)
    w = (torch.randn(16, 64, generator=gen) / 8).to(device)
    keys = torch.randn(16, 32768, 128, generator=gen).to(torch.bfloat16).to(device)
    return "dense", lambda: decode.indexer_topk(q, w, keys, 2048)


def _c5(device):
    from . import decode

    gen = torch.Generator().manual_seed(1582)
    q = (torch.randn(4, 64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16).to(device)
    w = (torch.randn(4, 64, generator=gen) / 8).to(device)
    raw = torch.randn(4, 131072, 128, generator=gen)
    scales = raw.reshape(4, 1024, 128 * 128).abs().amax(dim=2) / 448
    keys = (raw / scales.repeat_interleave(128, dim=1)[..., None]).to(torch.float8_e4m3fn).to(device)
    scales = scales.to(device)
    return "dense", lambda: decode.indexer_topk(q, w, keys, 2048, key_scales=scales)


def _c3_static(device):
    from . import decode, temporal

    gen = torch.Generator().manual_seed(1582)
    keys = torch.randn(4, 16385, 128, generator=gen).to(torch.bfloat16).to(device)
    q0 = torch.randn(4, 64, 128, generator=gen)
    q1 = 0.95 * q0 + math.sqrt(1 - 0.95**2) * torch.randn(4, 64, 128, generator=gen)
    q0, q1 = q0.to(torch.bfloat16).to(device), q1.to(torch.bfloat16).to(device)
    w = (torch.randn(4, 64, generator=gen) / 8).to(device)
    prev_top, prev_scores = decode.indexer_topk(q0, w, keys[:, :16384].contiguous(), 2048, return_scores=True)
    prev_max = temporal.block_max(prev_scores, 64)
    gamma = torch.full((4,), 0.25 * float(prev_scores.std()), device=device)
    return "static", lambda: temporal.temporal_step(q1, w, keys, prev_max, 16384, prev_top, gamma, block_size=64,
                                                    method="static")


def _c4_topk(device):
    from . import _lib as lib

    gen = torch.Generator().manual_seed(1582)
    t = 4096
    scores = torch.randn(t, t, generator=gen).mul_(0.1)
    scores = torch.where(torch.arange(t)[None, :] <= torch.arange(t)[:, None], scores,
                         torch.full_like(scores, -float("inf"))).to(device)
    visible = torch.arange(1, t + 1, dtype=torch.int32, device=device)
    idx = torch.empty(t, 512, dtype=torch.int64, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    return "topk", lambda: lib.call("dsa_topk", scores.data_ptr(), None, t, t, t, visible.data_ptr(), 512, 0,
                                    idx.data_ptr(), None, stream)


def _transition(device, fp8: bool):
    """One decode transition L - 1 -> L with AR(1) queries (rho 0.95): the
    keys, scales, weights, both queries, and the previous step's top-k and
    scores."""

    from . import decode

    gen = torch.Generator().manual_seed(1582)
    rows, length = 4, (131072 if fp8 else 16385)
    w = (torch.randn(rows, 64, generator=gen) / 8).to(device)
    raw = torch.randn(rows, length, 128, generator=gen)
    scales = None
    if fp8:
        scales = raw.reshape(rows, length // 128, 128 * 128).abs().amax(dim=2) / 448
        keys = (raw / scales.repeat_interleave(128, dim=1)[..., None]).to(torch.float8_e4m3fn).to(device)
        scales = scales.to(device).contiguous()
    else:
        keys = raw.to(torch.bfloat16).to(device)
    del raw
    q0 = torch.randn(rows, 64, 128, generator=gen) / math.sqrt(128)
    q1 = 0.95 * q0 + math.sqrt(1 - 0.95**2) * torch.randn(rows, 64, 128, generator=gen) / math.sqrt(128)
    q0, q1 = q0.to(torch.bfloat16).to(device), q1.to(torch.bfloat16).to(device)
    prev_top, prev_scores = decode.indexer_topk(q0, w, keys[:, : length - 1].contiguous(), 2048, key_scales=scales,
                                                return_scores=True)
    dense = decode.indexer_topk(q1, w, keys, 2048, key_scales=scales, return_scores=True)[1]
    sigma = (dense[:, : length - 1] - prev_scores).std(dim=1, unbiased=False)
    return keys, scales, w, q1, prev_top, prev_scores, sigma, length


def _c3_replay(device):
    from . import temporal

    keys, _, w, q1, prev_top, prev_scores, sigma, length = _transition(device, fp8=False)
    prev_max = temporal.block_max(prev_scores, 16)
    gamma = sigma.contiguous()
    return "replay", lambda: temporal.temporal_step(q1, w, keys, prev_max, length - 1, prev_top, gamma, block_size=16,
                                                    method="dynamic", scan_order="address", wave=33)


def _c5_replay(device):
    from . import temporal

    keys, scales, w, q1, prev_top, prev_scores, sigma, length = _transition(device, fp8=True)
    prev_max = temporal.block_max(prev_scores, 64)
    gamma = (0.25 * sigma).contiguous()
    return "replay", lambda: temporal.temporal_step(q1, w, keys, prev_max, length - 1, prev_top, gamma, block_size=64,
                                                    method="dynamic", scan_order="previous_hot", wave=96,
                                                    key_scales=scales)


def _c5_static(device):
    from . import temporal

    keys, scales, w, q1, prev_top, prev_scores, sigma, length = _transition(device, fp8=True)
    prev_max = temporal.block_max(prev_scores, 64)
    gamma = (0.25 * sigma).contiguous()
    return "static", lambda: temporal.temporal_step(q1, w, keys, prev_max, length - 1, prev_top, gamma, block_size=64,
                                                    method="static", key_scales=scales)


def _select_of(config):
    # The same decode step, timed by the list select's marks.
    def make(device):
        return "select", config(device)[1]
    return make


CONFIGS = {"c2": _c2, "c5": _c5, "c3-static": _c3_static, "c4-topk": _c4_topk,
           "c2-select": _select_of(_c2), "c5-select": _select_of(_c5), "c3-replay": _c3_replay, "c5-replay": _c5_replay,
           "c5-static": _c5_static}
KERNEL_SYMBOL["replay"] = "dsa_trace_temporal_resolve"


def replay_phases(log: np.ndarray, rows: int) -> dict:
    """Per-row totals of the replay's phases (rows r and 1024 + r of its log)."""

    us = lambda ticks: round(float(ticks) / WALL_CLOCK_MHZ, 2)  # noqa: E731
    out = {}
    for r in range(rows):
        a, tail = log[r], log[1024 + r]
        out[r] = {"setup_us": us(a[7]), "loop_us": us(a[0]), "decisions_us": us(a[1]), "exact_selects_us": us(a[2]),
                  "joins_us": us(a[4]), "cut_moves_us": us(a[5]), "exact_selects": int(a[3]) & 0xFFFFFFFF,
                  "cut_moves": int(a[3]) >> 32, "loop_steps": (int(a[6]) >> 24) & 0xFFFFFF,
                  "listed_keys": int(a[6]) & 0xFFFFFF, "tail_us": us(tail[0]), "tail_writeback_topk_us": us(tail[1]),
                  "tail_resets_us": us(tail[2])}
    return out


def timeline(config: str, runs: int = 8) -> dict:
    if not TRACE_LIBRARY.exists():
        raise RuntimeError(f"{TRACE_LIBRARY} is missing: run `python -m dsa_amd.build --trace` first")
    _lib.LIBRARY_PATH = TRACE_LIBRARY
    lib = _lib.load()
    device = torch.device("cuda", 0)
    kernel, step = CONFIGS[config](device)
    reader = getattr(lib, KERNEL_SYMBOL[kernel])
    reader.restype = ctypes.c_int
    reader.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32]
    n = 4096 * 8
    host = (ctypes.c_uint64 * n)()
    flush = torch.ones(512 * 1024 * 1024 // 4, device=device)
    for i in range(runs):
        torch.cuda.synchronize()
        if reader(host, n, 1) != 0:
            raise RuntimeError(lib.dsa_last_error().decode(errors="replace"))
        flush.amax()
        step()
        torch.cuda.synchronize()
    if reader(host, n, 0) != 0:
        raise RuntimeError(lib.dsa_last_error().decode(errors="replace"))
    log = np.frombuffer(host, dtype=np.uint64).reshape(4096, 8).astype(np.int64)
    if kernel == "replay":
        return {"config": config, "kernel": "replay", "rows": replay_phases(log, 4)}
    wgs = np.flatnonzero(log[:, 0] > 0)
    names = MARKS[kernel]
    raw = log[wgs][:, : len(names)].astype(np.float64)
    raw[raw == 0] = np.nan  # a mark the workgroup did not reach (an early exit)
    t = (raw - log[wgs, 0].min()) / WALL_CLOCK_MHZ  # microseconds
    out = {"config": config, "kernel": kernel, "workgroups": int(wgs.size), "unit": "us from the earliest start",
           "marks": {}}
    for i, name in enumerate(names):
        col = t[:, i][~np.isnan(t[:, i])]
        if col.size == 0:
            continue
        out["marks"][name] = {q: round(float(np.percentile(col, p)), 2)
                              for q, p in (("min", 0), ("p10", 10), ("median", 50), ("p90", 90), ("max", 100))}
        out["marks"][name]["workgroups"] = int(col.size)
    end = np.nanmax(t, axis=1)  # each workgroup's latest mark
    xcd = wgs % 8
    out["per_xcd_end"] = {int(x): {"median": round(float(np.median(end[xcd == x])), 2),
                                   "max": round(float(end[xcd == x].max()), 2)} for x in range(8)}
    return out


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--config", choices=sorted(CONFIGS), default="c2")
    parser.add_argument("--runs", type=int, default=8)
    parser.add_argument("--out", default=None)
    args = parser.parse_args()
    result = timeline(args.config, args.runs)
    text = json.dumps(result, indent=1)
    if args.out:
        Path(args.out).parent.mkdir(parents=True, exist_ok=True)
        Path(args.out).write_text(text)
    print(text, flush=True)


if __name__ == "__main__":
    sys.exit(main())
