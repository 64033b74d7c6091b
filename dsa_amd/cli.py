"""Command-line driver: collect score traces on the GPU and replay them.

Mirrors the reference's ``temporal-dsa analyze`` entry point (reference
cli.py:42-103): it finds ``.npz`` traces under ``--trace-roots``, replays each
with the sweep of the ``replay`` section of a YAML config (``k_values``,
``block_sizes``, ``gamma_sigma``, ``key_bytes``, ``metadata_bytes_per_block``,
optional ``calibrated_margins`` per layer, or a ``--margin-file``), and writes
``temporal_stats.csv``, ``block_stats.csv`` (reference cli.py:17-20,55-58,
replay.py:403-474), ``replay_rows.csv`` and the aggregated
``replay_summary.csv`` to ``--output``.  The replay and the statistics run in
the HIP kernels (:mod:`dsa_amd.replay`).  The reference's graphs, hardware
extrapolation and verdict report are analysis presentation and stay with the
reference's tools, which read the traces and CSVs written here.

``collect`` writes a synthetic decode trajectory's dense score trace (AR(1)
queries, N(0,1) keys, one key appended per step) in the reference's format:

    python -m dsa_amd.cli collect --output traces/synthetic.npz --length 16384 --steps 64
    python -m dsa_amd.cli analyze --trace-roots traces --output results --config configs.yaml
"""

from __future__ import annotations

import argparse
import json
import math
from pathlib import Path

import numpy as np
import yaml


def _trace_paths(roots: list[Path]) -> list[Path]:
    paths: list[Path] = []
    for root in roots:
        paths.extend([root] if root.is_file() and root.suffix == ".npz" else sorted(root.rglob("*.npz")))
    if not paths:
        raise FileNotFoundError("no .npz traces found")
    return paths


def analyze(args: argparse.Namespace) -> None:
    import pandas as pd

    from .replay import aggregate_rows, block_temporal_stats, replay_trace_rows, temporal_stats
    from .trace import load_trace

    config = yaml.safe_load(args.config.read_text(encoding="utf-8")) if args.config else {}
    replay = dict(config.get("replay", {}))
    if args.margin_file:
        payload = json.loads(args.margin_file.read_text(encoding="utf-8"))
        replay["calibrated_margins"] = {
            str(layer): {int(block): value for block, value in blocks.items()}
            for layer, blocks in payload["margins"].items()
        }
    k_values = replay.get("k_values", [2048])
    block_sizes = replay.get("block_sizes", [16, 32, 64, 128])
    gammas = replay.get("gamma_sigma", [0.0, 0.25, 0.5, 1.0])
    rows: list[dict] = []
    temporal_frames, block_frames = [], []
    for path in _trace_paths(args.trace_roots):
        trace = load_trace(path)
        temporal_frames.append(temporal_stats(trace, k_values))
        block_frames.append(block_temporal_stats(trace, block_sizes, k_values))
        margins = replay.get("calibrated_margins", {}).get(str(trace.layer))
        if margins:
            margins = {int(b): float(v) for b, v in margins.items()}
        rows.extend(replay_trace_rows(
            trace, k_values=k_values, block_sizes=block_sizes, gamma_sigma_values=gammas,
            key_bytes=replay.get("key_bytes", 256), metadata_bytes_per_block=replay.get("metadata_bytes_per_block", 8),
            absolute_margins=margins, wave=args.wave,
        ))
        print(f"replayed {path} ({trace.scores.shape[0] - 1} transitions)", flush=True)
    args.output.mkdir(parents=True, exist_ok=True)
    pd.concat(temporal_frames, ignore_index=True).to_csv(args.output / "temporal_stats.csv", index=False)
    pd.concat(block_frames, ignore_index=True).to_csv(args.output / "block_stats.csv", index=False)
    frame = pd.DataFrame(rows)
    frame.to_csv(args.output / "replay_rows.csv", index=False)
    aggregate_rows(frame).to_csv(args.output / "replay_summary.csv", index=False)
    print(f"wrote {len(frame)} rows to {args.output}", flush=True)


def collect(args: argparse.Namespace) -> None:
    import torch

    from .trace import collect_trace, save_trace

    gen = torch.Generator().manual_seed(args.seed)
    steps, length = args.steps, args.length
    device = torch.device("cuda", 0)
    keys = torch.randn(length + steps - 1, 128, generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn(64, generator=gen) / 8).to(device)
    q = torch.randn(64, 128, generator=gen) / math.sqrt(128)
    qs = []
    for _ in range(steps):
        qs.append(q.to(torch.bfloat16))
        q = args.rho * q + math.sqrt(1 - args.rho * args.rho) * torch.randn(64, 128, generator=gen) / math.sqrt(128)
    queries = torch.stack(qs).to(device)
    lengths = np.arange(length, length + steps)
    trace = collect_trace(queries, w, keys, lengths, layer=args.layer, workload="synthetic", prompt_id=str(args.seed),
                          metadata={"rho": args.rho, "seed": args.seed})
    save_trace(args.output, trace)
    print(f"wrote {args.output}: {steps} steps, lengths {length}..{length + steps - 1}", flush=True)


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(prog="dsa-amd")
    sub = parser.add_subparsers(dest="command", required=True)
    a = sub.add_parser("analyze", help="replay traces on the GPU and write the replay tables")
    a.add_argument("--trace-roots", type=Path, nargs="+", required=True)
    a.add_argument("--config", type=Path, default=None)
    a.add_argument("--output", type=Path, required=True)
    a.add_argument("--margin-file", type=Path)
    a.add_argument("--wave", type=int, default=1, help="blocks between dynamic threshold refreshes (1: the reference)")
    a.set_defaults(function=analyze)
    c = sub.add_parser("collect", help="write a synthetic decode trajectory's score trace")
    c.add_argument("--output", type=Path, required=True)
    c.add_argument("--length", type=int, default=16384)
    c.add_argument("--steps", type=int, default=64)
    c.add_argument("--rho", type=float, default=0.95)
    c.add_argument("--seed", type=int, default=1582)
    c.add_argument("--layer", type=int, default=0)
    c.set_defaults(function=collect)
    return parser


def main(argv: list[str] | None = None) -> None:
    args = build_parser().parse_args(argv)
    args.function(args)


if __name__ == "__main__":
    main()
