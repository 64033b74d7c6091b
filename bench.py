"""Headline benchmark: batched decode indexer scoring + top-K on one MI355X.

Workload: B=16 independent sequences, L=32768 bf16 keys
~ N(0,1) with 1% "hot" keys scaled x4, q bf16 ~ N(0,1)/sqrt(128), fp32 head
weights ~ N(0,1/64), exact top-K=2048 per sequence (stable_topk set
semantics).  One step = dense scores of all 16 x 32768 keys + the top-K of
every sequence, inputs resident in HBM.  Four distinct key sets (4 x 128 MiB)
are rotated so that the 256 MB last-level cache cannot hold the step's keys.

The timed region replays a HIP graph of up to 40 consecutive steps (the four
key sets in turn), sized to divide the number of timed steps: the step is two
kernel launches and Python issues them slower than the GPU runs them, and each
graph launch costs about as much as one step's gap between kernels, so a
longer graph leaves less of it per step.  Prints one JSON line (see the driver contract) with a
`roofline` object for the dominant kernel (the scoring kernel, timed by HIP
events that the kernel records at its own start and end, on the stream it
runs on; its bytes are the step's algorithmic bytes, keys + queries +
weights + top-K outputs, with the score write reported apart) and a `cpu_baseline`
object (the oracle's CPU restatement of the reference path timed on this host
on a bounded sample).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BATCH = 16
LENGTH = 32768
TOPK = 2048
ROTATIONS = 4
HOT_FRACTION = 0.01
SEED = 1582


def parse_args() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--config", choices=("c2", "c3", "c4", "c5", "progressive", "sidecar", "verifier", "replay"), default="c2",
                        help="c2: the headline decode step (default); c3: temporal replay over 256 decode steps; "
                        "c4: causal prefill indexer + top-512; c5: fp8 long-context decode; "
                        "progressive: the reference's method comparison (full / H8 / two-pass / fused); "
                        "sidecar: the indexer's query/key encoders at the decode and prefill shapes; "
                        "verifier: the live two-path verifier step against the dense step (C3 shape); "
                        "replay: the reference's trace replay sweep over a GPU-collected C3-shape trace")
    parser.add_argument("--out", default=None, help="c4/c5/progressive: also write the full table (JSON) here")
    parser.add_argument("--flush", choices=("read", "write"), default="read",
                        help="c4/c5/progressive: cache flush before each timed replay: read 512 MiB (default) or "
                        "add 1 to it as the reference does (leaves the last-level cache full of dirty lines)")
    parser.add_argument("--c3-out", default=None, help="c3: also write the per-variant table (JSON) here")
    parser.add_argument("--c3-blocks", default=",".join(map(str, C3_BLOCKS)), help="c3: block sizes to replay")
    parser.add_argument("--c3-wave1-blocks", default="64",
                        help="c3: block sizes that also replay the dynamic scans at the reference's per-block refresh")
    parser.add_argument("--c3-gamma", default=",".join(map(str, C3_GAMMA_SIGMA)), help="c3: gamma_sigma values")
    parser.add_argument("--c3-refreshes", type=int, default=32,
                        help="c3: threshold refreshes per dynamic scan (the reference refreshes after every block)")
    return parser.parse_args()


def make_inputs(device):
    import torch

    gen = torch.Generator(device=device).manual_seed(SEED)
    cpu_gen = torch.Generator().manual_seed(SEED)
    q = (torch.randn(BATCH, 64, 128, generator=gen, device=device) / math.sqrt(128)).to(torch.bfloat16)
    w = torch.randn(BATCH, 64, generator=gen, device=device) / 8.0
    key_sets = []
    hot = round(HOT_FRACTION * LENGTH)
    for _ in range(ROTATIONS):
        keys = torch.randn(BATCH, LENGTH, 128, generator=gen, device=device)
        for b in range(BATCH):
            idx = torch.randperm(LENGTH, generator=cpu_gen)[:hot].to(device)
            keys[b, idx] *= 4.0
        key_sets.append(keys.to(torch.bfloat16))
        del keys
    return q, w, key_sets


def host_cpu() -> dict:
    """Host facts the CPU baseline is quoted with: online CPUs (nproc), the
    CPUs this process may run on, and the processor model name."""

    import os

    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "model": model}


def _percentile(sorted_values, frac: float) -> float:
    pos = frac * (len(sorted_values) - 1)
    lo = int(pos)
    hi = min(lo + 1, len(sorted_values) - 1)
    return sorted_values[lo] + (sorted_values[hi] - sorted_values[lo]) * (pos - lo)


def cpu_baseline(q, w, keys, k: int, budget_s: float) -> tuple[dict, "object"]:
    """Oracle restatement of the reference CPU path: torch fp32 dense score
    (reference progressive_kernel.py:45-55) + numpy stable_topk (metrics.py:9-22).

    Protocol: one run = one sequence (L keys) scored + its stable top-K.  5
    warm-up runs, then at least 20 timed runs (more while the budget lasts),
    at all host threads this process may use and at 1 thread; median, p5 and
    p95 of each, keys/s = L / median run time."""

    import torch

    from oracle import scores as S
    from oracle import topk as T

    host = host_cpu()
    # The GPU box caps a job's threads through OMP_NUM_THREADS; use that share
    # (or every CPU this process may run on, when it is unset).
    all_threads = min(int(os.environ.get("OMP_NUM_THREADS", host["affinity"])), host["affinity"])
    q0, w0, k0 = q[0].cpu(), w[0].cpu(), keys[0].cpu()
    saved = torch.get_num_threads()
    top = None
    legs = {}
    try:
        for name, threads in (("all", all_threads), ("one", 1)):
            torch.set_num_threads(threads)
            for _ in range(5):
                top = T.stable_topk(S.torch_full_scores(q0, w0, k0).numpy(), k)
            times = []
            start = time.perf_counter()
            while len(times) < 20 or time.perf_counter() - start < budget_s / 2:
                t0 = time.perf_counter()
                top = T.stable_topk(S.torch_full_scores(q0, w0, k0).numpy(), k)
                times.append(time.perf_counter() - t0)
                if len(times) >= 20 and time.perf_counter() - start >= budget_s / 2:
                    break
            times.sort()
            med = _percentile(times, 0.5)
            legs[name] = {
                "threads": threads,
                "runs": len(times),
                "median_ms": round(med * 1e3, 3),
                "p5_ms": round(_percentile(times, 0.05) * 1e3, 3),
                "p95_ms": round(_percentile(times, 0.95) * 1e3, 3),
                "g_keys_per_s": round(LENGTH / med / 1e9, 5),
            }
    finally:
        torch.set_num_threads(saved)
    info = {
        "value": legs["all"]["g_keys_per_s"],
        "unit": "G keys/s",
        "cores": all_threads,
        "kind": "port",
        "sample": f"1 sequence (L={LENGTH}, K={k}) scored + stable_topk per run; 5 warm-up + "
                  f"{legs['all']['runs']} timed runs at {all_threads} threads, {legs['one']['runs']} at 1 thread; "
                  f"value = L / median run",
        "one_thread": legs["one"],
        "all_threads": legs["all"],
        "nproc": host["nproc"],
        "affinity_cpus": host["affinity"],
        "cpu_model": host["model"],
    }
    return info, top


def main() -> None:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build (the path shards by sequence, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    if args.config == "c3":
        run_c3(args)
        return
    if args.config in ("c4", "c5", "progressive", "sidecar", "verifier", "replay"):
        {"c4": run_c4, "c5": run_c5, "progressive": run_progressive, "sidecar": run_sidecar,
         "verifier": run_verifier, "replay": run_replay}[args.config](args)
        return
    import torch

    from dsa_amd import _lib, metrics

    _lib.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    q, w, key_sets = make_inputs(device)
    scores = torch.empty(BATCH, LENGTH, device=device, dtype=torch.float32)
    out_idx = torch.empty(BATCH, TOPK, device=device, dtype=torch.int64)
    ws_bytes = int(_lib.query("dsa_score_topk_workspace_bytes", BATCH, LENGTH))
    workspace = torch.zeros(ws_bytes, device=device, dtype=torch.uint8)
    # The decode step = dsa_score_topk, issued as its two halves so that the
    # scoring kernel (the dominant one) can be timed on its own.  Launches go
    # to torch's current stream (the capture stream while a graph records).
    def score(keys):
        _lib.call(
            "dsa_score_hist", q.data_ptr(), w.data_ptr(), keys.data_ptr(), None, scores.data_ptr(),
            BATCH, LENGTH, TOPK, _lib.DTYPE_BF16, workspace.data_ptr(), ws_bytes,
            torch.cuda.current_stream().cuda_stream,
        )

    def select():
        _lib.call(
            "dsa_select_topk", scores.data_ptr(), BATCH, LENGTH, TOPK, out_idx.data_ptr(), None,
            workspace.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream,
        )

    for i in range(args.warmup):
        score(key_sets[i % ROTATIONS])
        select()
    torch.cuda.synchronize()

    # The step is launch-bound from Python (two kernels, ~40 us of GPU work),
    # so the timed region replays a HIP graph of consecutive steps (the key
    # sets in turn); every launch in it is one of the library's kernels.  The
    # graph holds the largest of 40, 20, 12, 8 steps that divides the timed
    # steps (else 4, and the timed steps round up to a multiple of 4): a
    # graph launch costs about one step's kernel gap, about 1 us per step
    # over a graph of 4 steps against 40.
    per_graph = next((n for n in (40, 20, 12, 8, 4) if args.steps % n == 0), ROTATIONS)
    graph = torch.cuda.CUDAGraph()
    capture = torch.cuda.Stream(device)
    capture.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(capture):
        for r in range(ROTATIONS):  # warm the capture stream
            score(key_sets[r])
            select()
    torch.cuda.current_stream(device).wait_stream(capture)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for i in range(per_graph):
            score(key_sets[i % ROTATIONS])
            select()
    replays = max(1, -(-args.steps // per_graph))
    steps = replays * per_graph
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record(stream)
    for _ in range(replays):
        graph.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / steps
    keys_per_step = BATCH * LENGTH
    value = keys_per_step / (ms_per_step / 1e3) / 1e9

    # Per-kernel durations: HIP events around each launch, eagerly, on the
    # stream the kernels run on.
    # Per-kernel durations: the timed variants of the two halves have their
    # kernels record HIP events at their own start and end (hipExtLaunchKernel),
    # on the stream they run on, so each interval is the kernels' execution
    # alone, as rocprofv3's kernel trace reports it.
    # The launches queue behind a hold on the stream (a bounded spin kernel
    # sized to outlast their issue), so that they run back to back as in the
    # graph replays instead of paced by the host's calls.
    timed = max(20, min(args.steps, 100))
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(4 * timed)]
    for m in marks:  # the events must exist before a launch records them
        m.record(stream)
    torch.cuda.synchronize()
    hold = stream_hold(stream, 2.0 + 0.06 * timed)
    hold()
    for i in range(timed):
        keys = key_sets[i % ROTATIONS]
        _lib.call(
            "dsa_score_hist_timed", q.data_ptr(), w.data_ptr(), keys.data_ptr(), None, scores.data_ptr(),
            BATCH, LENGTH, TOPK, _lib.DTYPE_BF16, workspace.data_ptr(), ws_bytes, stream.cuda_stream,
            marks[4 * i].cuda_event, marks[4 * i + 1].cuda_event,
        )
        _lib.call(
            "dsa_select_topk_timed", scores.data_ptr(), BATCH, LENGTH, TOPK, out_idx.data_ptr(), None,
            workspace.data_ptr(), ws_bytes, stream.cuda_stream, marks[4 * i + 2].cuda_event,
            marks[4 * i + 3].cuda_event,
        )
    torch.cuda.synchronize()
    score_ms = [marks[4 * i].elapsed_time(marks[4 * i + 1]) for i in range(timed)]
    topk_ms = [marks[4 * i + 2].elapsed_time(marks[4 * i + 3]) for i in range(timed)]
    # idle time between one step's selection and the next step's scoring: near
    # zero when the launches ran back to back behind the hold
    gaps = sorted(marks[4 * i + 3].elapsed_time(marks[4 * i + 4]) * 1e3 for i in range(timed - 1))
    gap_us = gaps[len(gaps) // 2]

    # Algorithmic bytes per step, the measurement contract's figure: every key
    # row once (256 B), the query block and weights once per sequence, and
    # the K (index, score) outputs of each row, 134,746,112 B at C2.  The
    # roofline divides them by the scoring kernel's average duration.  The
    # fp32 score row the scoring kernel writes (4 B per key) is not counted:
    # it is reported on its own as score_write_bytes.
    step_bytes = keys_per_step * 256 + BATCH * (64 * 128 * 2 + 64 * 4) + BATCH * TOPK * (4 + 4)
    score_write_bytes = keys_per_step * 4
    score_avg_ms = sum(score_ms) / len(score_ms)
    achieved = step_bytes / (score_avg_ms / 1e3) / 1e9
    # HBM bytes per launch of the scoring kernel, from the committed rocprofv3
    # FETCH_SIZE / WRITE_SIZE passes (scaled by a copy kernel of known size).
    traffic = None
    traffic_file = ROOT / "profiles" / "dense_scores_c2_traffic.json"
    if traffic_file.exists():
        traffic = json.loads(traffic_file.read_text()).get("traffic_bytes")
    # Measured streaming ceiling: a read-only launch with the scoring kernel's
    # grid and load pattern over the same key sets, timed like the scoring
    # kernel (events the kernel records at its own start and end).
    sink = torch.empty(256, device=device, dtype=torch.float32)
    key_bytes = keys_per_step * 256
    smarks = [torch.cuda.Event(enable_timing=True) for _ in range(2 * timed)]
    for m in smarks:
        m.record(stream)
    torch.cuda.synchronize()
    hold()
    for i in range(timed):
        _lib.call("dsa_stream_read", key_sets[i % ROTATIONS].data_ptr(), key_bytes, 256, sink.data_ptr(),
                  stream.cuda_stream, smarks[2 * i].cuda_event, smarks[2 * i + 1].cuda_event)
    torch.cuda.synchronize()
    stream_us = sum(smarks[2 * i].elapsed_time(smarks[2 * i + 1]) for i in range(timed)) * 1e3 / timed
    stream_gbs = key_bytes / (stream_us * 1e-6) / 1e9

    # Parity of one sequence against the oracle (Recall@K of the GPU set).
    baseline = None
    recall = None
    if not args.no_cpu_baseline:
        score(key_sets[0])
        select()
        torch.cuda.synchronize()
        baseline, cpu_top = cpu_baseline(q, w, key_sets[0], TOPK, args.cpu_seconds)
        recall = metrics.topk_recall(out_idx[0].cpu().numpy(), cpu_top)

    line = {
        "metric": "G keys scored/s + % HBM roofline, B=16 L=32K bf16 top-K2048; Recall@K",
        "value": round(value, 3),
        "unit": "G keys/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "C2 batched decode: B=16 x L=32768 bf16 keys (1% hot x4), 64x128 indexer, fp32 weights, exact top-K=2048 per sequence, 4 rotated key sets",
            "batch": BATCH,
            "length": LENGTH,
            "topk": TOPK,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "dense_scores_kernel<bf16, M=4, hist, lists>",
            "kernel_avg_us": round(score_avg_ms * 1e3, 3),
            "algorithmic_bytes": step_bytes,
            "score_write_bytes": score_write_bytes,
            "measured_peak": round(stream_gbs, 1),
            "frac_of_measured": round(achieved / stream_gbs, 4),
            "measured_peak_kernel": f"dsa_stream_read: the same {key_bytes} key bytes, grid and load pattern, "
            f"read only ({stream_us:.2f} us per launch)",
        },
        "step": {
            "score_us": round(score_avg_ms * 1e3, 3),
            "topk_us": round(sum(topk_ms) / len(topk_ms) * 1e3, 3),
            "algorithmic_bytes": step_bytes,
            "hbm_frac": round(step_bytes / (ms_per_step / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "wall_s": round(wall, 3),
            "timing": f"value: HIP events around {replays} replays of a graph of {per_graph} steps "
                      f"(the {ROTATIONS} key sets in turn); "
            f"score_us/topk_us: HIP events recorded by the kernels themselves (hipExtLaunchKernel) over {timed} eager steps "
            "queued behind a hold on the stream, so they run back to back",
            "launch_gap_us": round(gap_us, 3),
        },
        "recall_at_k": recall,
        "cpu_baseline": baseline,
    }
    print(json.dumps(line), flush=True)

# --------------------------------------------------------------------------
# C3: temporal replay over a decode trajectory
# --------------------------------------------------------------------------
C3_BATCH = 4
C3_LENGTH = 16384
C3_STEPS = 256
C3_TOPK = 2048
C3_RHO = 0.95
C3_BLOCKS = (16, 32, 64, 128)
C3_GAMMA_SIGMA = (0.0, 0.25, 0.5, 1.0)
# replay variants (reference replay.py:533-541, without the oracle order)
C3_REPLAY = (("static", "address"), ("static_hot_first", "previous_hot"), ("dynamic", "address"),
             ("dynamic", "previous_hot"), ("dynamic", "upper_hot"))
C3_HEADLINE_RECALL = 0.999  # headline: most bytes skipped among variants at this mean Recall@K or better


def c3_wave(blocks: int, block_size: int, refreshes: int) -> int:
    """Blocks per threshold refresh: about `refreshes` refreshes per scan,
    within the step's merge limit (k + wave * block_size <= 8192)."""

    return max(1, min(-(-blocks // refreshes), (8192 - C3_TOPK) // block_size))


def c3_inputs(device):
    """B=4 sequences: keys ~ N(0,1) bf16 for the final context, AR(1) queries
    q_t = rho q_{t-1} + sqrt(1 - rho^2) eps (eps ~ N(0,1)/sqrt(128)), fixed
    weights ~ N(0, 1/64); seeded CPU generator."""

    import torch

    gen = torch.Generator().manual_seed(SEED)
    total = C3_LENGTH + C3_STEPS - 1
    keys = torch.randn(C3_BATCH, total, 128, generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn(C3_BATCH, 64, generator=gen) / 8.0).to(device)
    q = torch.randn(C3_BATCH, 64, 128, generator=gen) / math.sqrt(128)
    queries = []
    for _ in range(C3_STEPS):
        queries.append(q.to(torch.bfloat16).to(device))
        q = C3_RHO * q + math.sqrt(1 - C3_RHO * C3_RHO) * torch.randn(C3_BATCH, 64, 128, generator=gen) / math.sqrt(128)
    return keys, w, queries


def c3_summary(rows: list[dict]) -> dict:
    """Aggregates as the reference's replay_trace (replay.py:592-627):
    medians of reductions, means of recall and exact match."""

    import numpy as np

    col = lambda name: np.asarray([r[name] for r in rows], dtype=np.float64)  # noqa: E731
    return {
        "transitions": len(rows),
        "qk_reduction": float(np.median(col("qk_reduction"))),
        "qk_reduction_p5": float(np.quantile(col("qk_reduction"), 0.05)),
        "net_byte_reduction": float(np.median(col("net_byte_reduction"))),
        "loaded_byte_reduction": float(np.median(col("loaded_byte_reduction"))),
        "recall": float(np.mean(col("recall"))),
        "recall_min": float(np.min(col("recall"))),
        "exact_match": float(np.mean(col("exact_match"))),
        "false_cold_blocks": int(np.sum(col("false_cold_blocks"))),
        "us_per_step": float(np.median(col("us"))),
    }


def run_c3(args) -> None:
    """BASELINE config 3 on one GPU: 256 decode steps of B=4 sequences whose
    context grows from 16384 keys by one key per step, K=2048.

    Every step is run dense (scores + exact top-k: the truth) and pruned.
    Replay variants are teacher-forced as the reference's replay_trace
    (replay.py:476-590): step t's pruned scan is seeded with the dense top-k
    of step t-1 and bounded by its block maxima + gamma_sigma * sigma_t
    (sigma_t = std of the score drift over the common keys).  Own-trajectory
    variants (approx.py:129-364) carry their own device state from step 0 with
    an absolute gamma fixed at gamma_sigma * sigma_1.  Bytes read per pruned
    step = keys scored x 256 + blocks x 8 (replay.py:369-371).
    """

    import numpy as np
    import torch

    from dsa_amd import _lib, approx, certified, decode, temporal

    _lib.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    keys, w, queries = c3_inputs(device)
    stream = torch.cuda.current_stream(device)
    lengths = [C3_LENGTH + t for t in range(C3_STEPS)]

    # Dense trajectory: scores and exact top-k of every step, timed per step.
    dense_scores, dense_topk, dense_us = [], [], []
    for t, length in enumerate(lengths):
        view = keys[:, :length].contiguous()
        for _ in range(2 if t == 0 else 1):  # the first call warms the workspace
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            top, sc = decode.indexer_topk(queries[t], w, view, C3_TOPK, return_scores=True)
            e1.record(stream)
        dense_scores.append(sc)
        dense_topk.append(top)
        torch.cuda.synchronize()
        dense_us.append(e0.elapsed_time(e1) * 1e3)
        del view
    sigma = [None] + [
        (dense_scores[t][:, : lengths[t - 1]] - dense_scores[t - 1]).std(dim=1, unbiased=False) for t in range(1, C3_STEPS)
    ]

    def true_mask(t):
        mask = torch.zeros(C3_BATCH, lengths[t], dtype=torch.bool, device=device)
        mask.scatter_(1, dense_topk[t], True)
        return mask

    truth = [true_mask(t) for t in range(C3_STEPS)]

    def record(rows, t, bs, step, us, dynamic=False):
        # Key rows loaded: a dynamic step's rounds also load the blocks they
        # score and then prune (temporal.keys_loaded); a static step loads the
        # keys it scores.
        length = lengths[t]
        nb = -(-length // bs)
        loaded = (temporal.keys_loaded(step, bs) if dynamic else step.qk_scored).to(torch.float64).cpu().numpy()
        hits = truth[t].gather(1, step.topk).sum(dim=1)
        true_blocks = torch.zeros(C3_BATCH, nb, dtype=torch.bool, device=device)
        true_blocks.scatter_(1, dense_topk[t] // bs, True)
        false_cold = (true_blocks & ~step.evaluated_blocks).sum(dim=1)
        qk = step.qk_scored.to(torch.float64)
        hits, false_cold, qk = hits.cpu().numpy(), false_cold.cpu().numpy(), qk.cpu().numpy()
        for b in range(C3_BATCH):
            rows.append({
                "qk_reduction": 1.0 - qk[b] / length,
                "net_byte_reduction": 1.0 - (qk[b] * 256 + nb * 8) / (length * 256),
                "loaded_byte_reduction": 1.0 - (loaded[b] * 256 + nb * 8) / (length * 256),
                "recall": hits[b] / C3_TOPK,
                "exact_match": float(hits[b] == C3_TOPK),
                "false_cold_blocks": int(false_cold[b]),
                "us": us,
            })

    def timed(fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        out = fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return out, e0.elapsed_time(e1) * 1e3

    variants = []
    wall0 = time.perf_counter()
    blocks_run = [int(x) for x in args.c3_blocks.split(",")]
    gammas_run = [float(x) for x in args.c3_gamma.split(",")]
    for bs in blocks_run:
        prev_max = [temporal.block_max(sc, bs) for sc in dense_scores[:-1]]
        wave = c3_wave(-(-lengths[-1] // bs), bs, args.c3_refreshes)
        for gamma_sigma in gammas_run:
            for method, order in C3_REPLAY:
                rows = []
                for t in range(1, C3_STEPS):
                    gamma = gamma_sigma * sigma[t]
                    step, us = timed(lambda: temporal.temporal_step(
                        queries[t], w, keys[:, : lengths[t]], prev_max[t - 1], lengths[t - 1], dense_topk[t - 1], gamma,
                        block_size=bs, method=method, scan_order=order, wave=wave))
                    record(rows, t, bs, step, us, dynamic=method == "dynamic")
                variants.append({"kind": "replay", "block_size": bs, "method": method, "scan_order": order,
                                 "gamma_sigma": gamma_sigma, "wave": wave if method == "dynamic" else 0,
                                 **c3_summary(rows)})
        # The reference's own schedule: the dynamic threshold refreshed after
        # every block (wave 1, replay.py:218-219), for the block sizes asked.
        wave1 = bs in [int(x) for x in args.c3_wave1_blocks.split(",") if x]
        if wave1:
            for gamma_sigma in gammas_run:
                for method, order in (("dynamic", "address"), ("dynamic", "previous_hot")):
                    rows = []
                    for t in range(1, C3_STEPS):
                        gamma = gamma_sigma * sigma[t]
                        step, us = timed(lambda: temporal.temporal_step(
                            queries[t], w, keys[:, : lengths[t]], prev_max[t - 1], lengths[t - 1], dense_topk[t - 1],
                            gamma, block_size=bs, method=method, scan_order=order, wave=1))
                        record(rows, t, bs, step, us, dynamic=True)
                    variants.append({"kind": "replay", "block_size": bs, "method": method, "scan_order": order,
                                     "gamma_sigma": gamma_sigma, "wave": 1, **c3_summary(rows)})
        # Certified bound (reference certified.py:18-62): U_b = previous block
        # max + the certified margin of the block (radius + fp32 rounding
        # allowance, dsa_certified_margins), computed per step from the two
        # queries and the keys; the margins are part of the timed step.
        certified_scans = [("static", "address", 0), ("dynamic", "previous_hot", wave)]
        if wave1:
            certified_scans.append(("dynamic", "previous_hot", 1))
        for method, order, cwave in certified_scans:
            rows = []
            for t in range(1, C3_STEPS):
                def certified_step():
                    margins = certified.certified_margins(queries[t], queries[t - 1], w, w, keys, lengths[t - 1], bs)
                    return temporal.temporal_step(
                        queries[t], w, keys[:, : lengths[t]], prev_max[t - 1], lengths[t - 1], dense_topk[t - 1], 0.0,
                        block_size=bs, method=method, scan_order=order, wave=cwave or wave, block_margins=margins)
                step, us = timed(certified_step)
                record(rows, t, bs, step, us, dynamic=method == "dynamic")
            variants.append({"kind": "certified", "block_size": bs, "method": method, "scan_order": order,
                             "gamma_sigma": "certified", "wave": cwave, **c3_summary(rows)})
        # Own trajectory: the policy state is initialised from the dense step 0
        # and then only sees what its own pruned steps scored.
        own = (
            approx.ApproxPolicy("dynamic_previous_max", dynamic_threshold=True, order="previous_max"),
            approx.ApproxPolicy("dynamic_previous_max_streak0", dynamic_threshold=True, order="previous_max",
                                cold_streak=0),
        )
        for policy in own:
            for gamma_sigma in gammas_run:
                state = approx.initialize_state(dense_scores[0], k=C3_TOPK, block_size=bs,
                                                capacity=lengths[-1])
                gamma = (gamma_sigma * sigma[1]).to(torch.float64)
                rows = []
                for t in range(1, C3_STEPS):
                    step, us = timed(lambda: approx.approx_step(
                        state, queries[t], w, keys[:, : lengths[t]], policy=policy, step=t, wave=wave, gamma=gamma))
                    record(rows, t, bs, step, us, dynamic=policy.dynamic_threshold)
                variants.append({"kind": "own", "block_size": bs, "method": policy.name, "scan_order": policy.order,
                                 "gamma_sigma": gamma_sigma, "wave": wave, **c3_summary(rows)})
        print(f"c3: block {bs} done ({time.perf_counter() - wall0:.1f} s)", file=sys.stderr, flush=True)

    eligible = [v for v in variants if v["recall"] >= C3_HEADLINE_RECALL]
    head = max(eligible, key=lambda v: (v["loaded_byte_reduction"], v["recall"]))
    dense_bytes = sum(C3_BATCH * length * 256 for length in lengths[1:])

    # GPU time of one step with the host's work hidden: the launches are
    # queued behind a 512 MiB read flush (as the C4/C5 legs time them), on the
    # last transition, for the dense step, the static step (block 64,
    # gamma_sigma 0.25) and the headline variant when it is a replay variant.
    flush = make_flush(args, device)
    t = C3_STEPS - 1
    view = keys[:, : lengths[t]].contiguous()

    def replay_fn(bs, method, order, gs, wave):
        pm = temporal.block_max(dense_scores[t - 1], bs)
        gamma = gs * sigma[t]
        return lambda i: temporal.temporal_step(queries[t], w, view, pm, lengths[t - 1], dense_topk[t - 1], gamma,
                                                block_size=bs, method=method, scan_order=order, wave=max(wave, 1))

    queued = {"dense": lambda i: decode.indexer_topk(queries[t], w, view, C3_TOPK),
              "static_block64": replay_fn(64, "static", "address", 0.25, 0)}
    if head["kind"] == "replay":
        queued["headline"] = replay_fn(head["block_size"], head["method"], head["scan_order"], head["gamma_sigma"],
                                       head["wave"])
    queued_us = {name: time_stats(graph_times(fn, 1, flush, 5, 30, device)) for name, fn in queued.items()}
    line = {
        "metric": "C3 temporal replay: key bytes skipped vs dense + Recall@K, B=4, 256 steps, L 16384->16639, K=2048",
        "value": round(head["loaded_byte_reduction"], 4),
        "unit": "fraction of dense key bytes not loaded (median over transitions)",
        "n_gpus": 1,
        "steps": C3_STEPS,
        "warmup": 0,
        "ms_per_step": round(head["us_per_step"] / 1e3, 5),
        "recall_at_k": round(head["recall"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "C3 temporal replay: B=4 x 256 decode steps, keys N(0,1) bf16, AR(1) queries rho=0.95, "
            "K=2048, blocks 16/32/64/128, gamma_sigma 0/0.25/0.5/1 and the certified radius",
            "headline_rule": "largest median reduction of the key bytes loaded (key rows loaded x 256 + blocks x 8) "
                             f"among variants with mean Recall@K >= {C3_HEADLINE_RECALL}; net_byte_reduction is the "
                             "reference's accounting from the keys scored (replay.py:369-371)",
            "refreshes_per_scan": args.c3_refreshes,
        },
        "headline": head,
        "dense": {"us_per_step": float(np.median(dense_us)), "bytes_equivalent": dense_bytes},
        "queued_gpu_us": {name: st["median_us"] for name, st in queued_us.items()},
        "queued_timing": "last transition, launches queued behind a 512 MiB read flush, median of 30 (the per-step "
                         "us above are eager: host work included)",
        "variants": len(variants),
        "wall_s": round(time.perf_counter() - wall0, 1),
    }
    if args.c3_out:
        Path(args.c3_out).parent.mkdir(parents=True, exist_ok=True)
        Path(args.c3_out).write_text(json.dumps({"line": line, "variants": variants}, indent=1))
    print(json.dumps(line), flush=True)


# --------------------------------------------------------------------------
# Shared: graph-replay timing with a cache flush outside the timed interval
# --------------------------------------------------------------------------
def graph_times(launch, variants: int, flush, warmup: int, measure: int, device) -> list:
    """Per-iteration milliseconds of launch(i), variant i round-robin, with a
    cache flush before each start event (reference benchmark_progressive_dsa.py:
    48-69).  The launches are issued eagerly: the flush keeps the GPU busy for
    ~150 us while the start event, the launches and the end event are queued
    behind it, so the interval holds the GPU work alone.  (A HIP graph replay
    queued the same way added ~10 us of launch latency to every interval.)"""

    import torch

    for it in range(warmup):
        flush()
        launch(it % variants)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(measure)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(measure)]
    for it in range(measure):
        flush()
        starts[it].record(stream)
        launch(it % variants)
        ends[it].record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in zip(starts, ends)]


def time_stats(values: list) -> dict:
    """Reference benchmark_progressive_dsa.py:37-45, in microseconds."""

    import numpy as np

    arr = np.asarray(values, dtype=np.float64) * 1e3
    return {"median_us": round(float(np.median(arr)), 3), "p5_us": round(float(np.percentile(arr, 5)), 3),
            "p95_us": round(float(np.percentile(arr, 95)), 3), "mean_us": round(float(arr.mean()), 3),
            "std_us": round(float(arr.std()), 3)}


def write_table(args, line: dict, rows: list) -> None:
    if args.out:
        Path(args.out).parent.mkdir(parents=True, exist_ok=True)
        Path(args.out).write_text(json.dumps({"line": line, "rows": rows}, indent=1))


FLUSH_BYTES = 512 * 1024 * 1024  # twice the 256 MB last-level cache


def stream_hold(stream, ms: float):
    """A callable that occupies `stream` for about `ms` milliseconds with a
    bounded spin kernel (torch.cuda._sleep), so that launches issued behind it
    queue up and then run back to back.  The spin's cycles per millisecond are
    measured once here."""

    import torch

    probe = 2_000_000
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(probe // 10)  # first launch outside the measurement
    e0.record(stream)
    torch.cuda._sleep(probe)
    e1.record(stream)
    torch.cuda.synchronize()
    per_ms = probe / max(e0.elapsed_time(e1), 1e-3)
    cycles = int(min(per_ms * ms, 50 * probe))
    return lambda: torch.cuda._sleep(cycles)


def make_flush(args, device):
    """A callable that evicts the inputs from every cache level: a read of
    512 MiB (default), or the reference's in-place add (benchmark_progressive_dsa.py:
    67), which also leaves the last-level cache full of dirty lines that the
    next kernel's misses must write back."""

    import torch

    buf = torch.ones(FLUSH_BYTES // 4, device=device, dtype=torch.float32)
    if args.flush == "write":
        return lambda: buf.add_(1)
    return lambda: buf.amax()


# --------------------------------------------------------------------------
# C4: causal multi-query (prefill) indexer, 8 layers, top-512 per query
# --------------------------------------------------------------------------
C4_T = 4096
C4_LAYERS = 8
C4_TOPK = 512
MFMA_BF16_PEAK_TFLOPS = 2500.0


def run_c4(args) -> None:
    """T=4096 queries x L=4096 causal keys per layer, 8
    independent layers, bf16 ~ N(0,1)/sqrt(128) queries and keys, fp32
    weights ~ N(0,1/64); per layer the causal score matrix and every
    query's top-512 over its visible keys in one launch
    (dsa_score_queries_topk); the scoring alone (dsa_score_queries) and the
    separate select (dsa_topk with row lengths) are timed beside it.  MFMA
    work = 64 heads x 128 dims x 2 FLOP per visible pair."""

    import torch

    from dsa_amd import _lib

    _lib.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    gen = torch.Generator().manual_seed(SEED)
    layers = []
    for _ in range(C4_LAYERS):
        q = (torch.randn(C4_T, 64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16).to(device)
        w = (torch.randn(C4_T, 64, generator=gen) / 8.0).to(device)
        keys = (torch.randn(C4_T, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16).to(device)
        layers.append((q, w, keys))
    scores = torch.empty(C4_T, C4_T, device=device, dtype=torch.float32)
    visible = torch.arange(1, C4_T + 1, dtype=torch.int32, device=device)
    idx = torch.empty(C4_T, C4_TOPK, device=device, dtype=torch.int64)

    def score(i):
        q, w, keys = layers[i]
        _lib.call("dsa_score_queries", q.data_ptr(), 64 * 128, w.data_ptr(), 64, None, 0, 64, keys.data_ptr(), C4_T,
                  C4_T, None, 0, scores.data_ptr(), C4_T, C4_T, C4_T, 0, _lib.DTYPE_BF16,
                  torch.cuda.current_stream().cuda_stream)

    def select(i):
        _lib.call("dsa_topk", scores.data_ptr(), None, C4_T, C4_T, C4_T, visible.data_ptr(), C4_TOPK, 0,
                  idx.data_ptr(), None, torch.cuda.current_stream().cuda_stream)

    def fused(i):
        q, w, keys = layers[i]
        _lib.call("dsa_score_queries_topk", q.data_ptr(), 64 * 128, w.data_ptr(), 64, keys.data_ptr(), C4_T, C4_T,
                  scores.data_ptr(), C4_T, C4_T, C4_T, 0, _lib.DTYPE_BF16, C4_TOPK, idx.data_ptr(), None, C4_TOPK,
                  torch.cuda.current_stream().cuda_stream)

    flush = make_flush(args, device)
    score_ms = graph_times(score, C4_LAYERS, flush, 5, 40, device)
    select_ms = graph_times(select, C4_LAYERS, flush, 5, 40, device)
    split_ms = graph_times(lambda i: (score(i), select(i)), C4_LAYERS, flush, 5, 40, device)
    step_ms = graph_times(fused, C4_LAYERS, flush, 5, 40, device)
    pairs = C4_T * (C4_T + 1) // 2
    flops = pairs * 64 * 128 * 2
    st = time_stats(step_ms)
    sc = time_stats(score_ms)
    achieved = flops / (sc["median_us"] * 1e-6) / 1e12
    line = {
        "metric": "C4 causal prefill indexer: TFLOP/s of the MFMA scoring + per-query top-512, T=L=4096, 8 layers",
        "value": round(flops / (st["median_us"] * 1e-6) / 1e12, 2),
        "unit": "TFLOP/s (scoring FLOPs over the layer step)",
        "n_gpus": 1,
        "steps": 40,
        "warmup": 5,
        "ms_per_step": round(st["median_us"] * C4_LAYERS / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "C4 prefill: T=4096 queries x L=4096 causal keys, 64x128 bf16, fp32 weights, "
                   "top-512 per query over its visible keys, 8 independent layers", "causal_pairs": pairs},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "prefill_scores_kernel<bf16> (multi-query, causal, dsa_score_queries)",
                     "kernel_median_us": sc["median_us"], "flops": flops},
        "layer": {"step": st, "score": sc, "topk": time_stats(select_ms), "split_step": time_stats(split_ms),
                  "topk_share_us": round(st["median_us"] - sc["median_us"], 3)},
        "step_kernel": "dsa_score_queries_topk: the scoring kernel with each query's top-512 selected by its wave "
                       "after its row is stored (split_step: dsa_score_queries then dsa_topk)",
        "timing": f"HIP events around one layer's launches, 512 MiB {args.flush} flush before each, median over 40",
    }
    write_table(args, line, [])
    print(json.dumps(line), flush=True)


# --------------------------------------------------------------------------
# C5: fp8 long-context decode
# --------------------------------------------------------------------------
C5_BATCH = 4
C5_LENGTH = 131072


def run_c5(args) -> None:
    """B=4 x L=131072 fp8 e4m3fn keys (one fp32 scale per
    128-key block, keys drawn around 10 Gaussian topic centroids), bf16
    queries, exact top-K=2048 per sequence (dsa_score_topk).  Three rotated
    key sets; HBM bytes per key 128 + 4/128 (scale)."""

    import torch

    from dsa_amd import _lib

    _lib.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    gen = torch.Generator().manual_seed(SEED)
    q = (torch.randn(C5_BATCH, 64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16).to(device)
    w = (torch.randn(C5_BATCH, 64, generator=gen) / 8.0).to(device)
    sets = []
    blocks = C5_LENGTH // 128
    for _ in range(3):
        centroids = torch.randn(C5_BATCH, 10, 128, generator=gen)
        topic = torch.randint(0, 10, (C5_BATCH, C5_LENGTH), generator=gen)
        raw = (torch.gather(centroids, 1, topic[..., None].expand(-1, -1, 128))
               + torch.randn(C5_BATCH, C5_LENGTH, 128, generator=gen)) / math.sqrt(2)
        scales = raw.reshape(C5_BATCH, blocks, 128 * 128).abs().amax(dim=2) / 448.0
        keys8 = (raw / scales.repeat_interleave(128, dim=1)[..., None]).to(torch.float8_e4m3fn)
        sets.append((keys8.to(device), scales.to(device).contiguous()))
        del raw
    scores = torch.empty(C5_BATCH, C5_LENGTH, device=device, dtype=torch.float32)
    idx = torch.empty(C5_BATCH, TOPK, device=device, dtype=torch.int64)
    ws_bytes = int(_lib.query("dsa_score_topk_workspace_bytes", C5_BATCH, C5_LENGTH))
    workspace = torch.zeros(ws_bytes, device=device, dtype=torch.uint8)

    def score(i):
        keys8, scales = sets[i]
        _lib.call("dsa_score_hist", q.data_ptr(), w.data_ptr(), keys8.data_ptr(), scales.data_ptr(), scores.data_ptr(),
                  C5_BATCH, C5_LENGTH, TOPK, _lib.DTYPE_FP8_E4M3, workspace.data_ptr(), ws_bytes,
                  torch.cuda.current_stream().cuda_stream)

    def select(i):
        _lib.call("dsa_select_topk", scores.data_ptr(), C5_BATCH, C5_LENGTH, TOPK, idx.data_ptr(), None,
                  workspace.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)

    flush = make_flush(args, device)
    step_ms = graph_times(lambda i: (score(i), select(i)), 3, flush, 10, 100, device)
    # The scoring kernel alone, after a flush: its timed variant has the kernel
    # record the events at its own start and end (hipExtLaunchKernel); the
    # select follows to keep the workspace consistent.
    score_ms = []
    side = torch.cuda.current_stream(device)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(side)
    e1.record(side)
    for it in range(60):
        flush()
        keys8, scales = sets[it % 3]
        _lib.call("dsa_score_hist_timed", q.data_ptr(), w.data_ptr(), keys8.data_ptr(), scales.data_ptr(),
                  scores.data_ptr(), C5_BATCH, C5_LENGTH, TOPK, _lib.DTYPE_FP8_E4M3, workspace.data_ptr(), ws_bytes,
                  side.cuda_stream, e0.cuda_event, e1.cuda_event)
        select(it % 3)
        torch.cuda.synchronize()
        if it >= 10:
            score_ms.append(e0.elapsed_time(e1))
    st = time_stats(step_ms)
    sc = time_stats(score_ms)
    keys_per_step = C5_BATCH * C5_LENGTH
    score_bytes = keys_per_step * (128 + 4) + C5_BATCH * (blocks * 4 + 64 * 128 * 2 + 64 * 4)
    progressive = c5_progressive(q, w, sets, idx, flush, device)
    temporal_leg = c5_temporal(q, w, sets, flush, device)
    achieved = score_bytes / (sc["median_us"] * 1e-6) / 1e9
    line = {
        "metric": "C5 fp8 long-context decode: G keys scored/s + % HBM roofline, B=4 L=131072 fp8 top-K2048",
        "value": round(keys_per_step / (st["median_us"] * 1e-6) / 1e9, 3),
        "unit": "G keys/s",
        "n_gpus": 1,
        "steps": 100,
        "warmup": 10,
        "ms_per_step": round(st["median_us"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 keys, bf16 queries",
        "data": "synthetic",
        "config": {"workload": "C5: B=4 x L=131072 fp8 e4m3fn keys (10 topic clusters, per-128-key fp32 scales), "
                   "64x128 indexer, exact top-K=2048, 3 rotated key sets"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "dense_scores_kernel<fp8, M=4, hist, lists>", "kernel_median_us": sc["median_us"],
                     "algorithmic_bytes": score_bytes},
        "step": st,
        "score": sc,
        "progressive": progressive,
        "temporal": temporal_leg,
        "timing": f"step: HIP events around the step's launches, 512 MiB {args.flush} flush before each, median over 100; "
                  "score: HIP events recorded by the scoring kernel itself (hipExtLaunchKernel), median over 50",
    }
    write_table(args, line, [])
    print(json.dumps(line), flush=True)


C5_TEMPORAL_GAMMA_SIGMA = (-0.25, 0.0, 0.25, 0.5, 1.0, 2.0, 3.0, 4.0)
C5_TEMPORAL_RHO = 0.95


def c5_temporal(q, w, sets, flush, device) -> dict:
    """C5 with block-64 temporal pruning, which skips key bytes: one decode
    step of the four sequences from L-1 to L = 131072 fp8 keys (the last key
    appended), the query drifting as AR(1) with rho 0.95 from the C5 query.
    Teacher-forced as the reference's replay (replay.py:225-400): seeds = the
    dense top-2048 of step L-1, U_b = its block maxima + gamma_sigma * sigma
    (sigma = std of the score drift), static (address) and dynamic
    (previous-hot, 22 threshold refreshes) scans.  Reports, per variant, the
    median step time (eager, after a cache flush), the key bytes read (key
    rows loaded x 128 + 128-key scales + 8 B of metadata per block; a dynamic
    step's rounds load the blocks they score and then prune as well, so its
    key rows loaded exceed its keys scored) against the dense step's, the
    same from the keys scored (the reference's accounting), and Recall@K
    against the dense top-2048.  The dynamic scan also runs at the
    reference's schedule, a refresh after every block (wave 1,
    replay.py:218-219), and every scan also with the certified margins
    (certified.py:18-48 over the fp8 keys, dsa_certified_margins, computed
    inside the timed step) in place of gamma."""

    import numpy as np
    import torch

    from dsa_amd import certified, decode, temporal

    block = 64
    keys8, scales = sets[0]
    gen = torch.Generator().manual_seed(SEED + 5)
    q_prev = q.float().cpu()
    q_now = (C5_TEMPORAL_RHO * q_prev + math.sqrt(1 - C5_TEMPORAL_RHO ** 2)
             * torch.randn(q_prev.shape, generator=gen) / math.sqrt(128)).to(torch.bfloat16).to(device)
    q_prev = q
    prev_len = C5_LENGTH - 1
    prev_top, prev_scores = decode.indexer_topk(q_prev, w, keys8[:, :prev_len], TOPK, key_scales=scales,
                                                return_scores=True)
    dense_top, dense = decode.indexer_topk(q_now, w, keys8, TOPK, key_scales=scales, return_scores=True)
    sigma = (dense[:, :prev_len] - prev_scores).std(dim=1, unbiased=False)
    prev_max = temporal.block_max(prev_scores, block)
    nb = C5_LENGTH // block
    truth = torch.zeros(C5_BATCH, C5_LENGTH, dtype=torch.bool, device=device)
    truth.scatter_(1, dense_top, True)
    dense_bytes = C5_LENGTH * 128 + (C5_LENGTH // 128) * 4
    variants = []
    stream = torch.cuda.current_stream(device)
    # the dynamic scan refreshes after the largest wave the step's merge allows
    # (k + wave * block <= 8192: 96 blocks, 22 refreshes per scan), or after
    # every block (the reference's schedule)
    scans = (("static", "address", 0), ("dynamic", "previous_hot", (8192 - TOPK) // block),
             ("dynamic", "previous_hot", 1))
    for (method, order, wave), gs in [(m, g) for m in scans for g in (*C5_TEMPORAL_GAMMA_SIGMA, "certified")]:
        gamma = 0.0 if gs == "certified" else gs * sigma

        def run():
            margins = None
            if gs == "certified":
                margins = certified.certified_margins(q_now, q_prev, w, w, keys8, prev_len, block,
                                                      key_scales=scales)
            return temporal.temporal_step(q_now, w, keys8, prev_max, prev_len, prev_top, gamma, block_size=block,
                                          method=method, scan_order=order, wave=max(wave, 1), key_scales=scales,
                                          block_margins=margins)

        times = []
        for it in range(12):
            flush()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            step = run()
            e1.record(stream)
            torch.cuda.synchronize()
            if it >= 2:
                times.append(e0.elapsed_time(e1) * 1e3)
        qk = step.qk_scored.double().cpu().numpy()
        # key rows loaded: a dynamic step's rounds also load the blocks they
        # score and then prune; a static step loads the keys it scores
        loaded = (temporal.keys_loaded(step, block) if method == "dynamic" else step.qk_scored).double().cpu().numpy()
        hits = truth.gather(1, step.topk).sum(dim=1).cpu().numpy()
        read = loaded * 128 + (C5_LENGTH // 128) * 4 + nb * 8
        scored_read = qk * 128 + (C5_LENGTH // 128) * 4 + nb * 8
        variants.append({
            "method": method, "scan_order": order, "wave": wave, "gamma_sigma": gs,
            "us_per_step": float(np.median(times)),
            "key_bytes_skipped": float(np.mean(1.0 - read / dense_bytes)),
            "key_bytes_skipped_scored": float(np.mean(1.0 - scored_read / dense_bytes)),
            "qk_reduction": float(np.mean(1.0 - qk / C5_LENGTH)),
            "recall": float(np.mean(hits / TOPK)),
        })
    eligible = [v for v in variants if v["recall"] >= 0.999]
    best = max(eligible, key=lambda v: v["key_bytes_skipped"]) if eligible else None
    return {"block_size": block, "rho": C5_TEMPORAL_RHO, "variants": variants, "best_at_recall_0.999": best}


def c5_progressive(q, w, sets, dense_idx, flush, device) -> dict:
    """C5 with block-64 progressive pruning: per sequence the fused H8 ->
    promote -> +56 heads kernel on the fp8 keys (direct blocks drawn as the
    reference's direct_mask at its 32K fraction, the promotion threshold at its
    0.10 target, benchmark_progressive_dsa.py:74-91), then the exact top-2048
    of the four rows (dsa_topk_distributed).  Reports the step time, Recall@K
    against the dense step's top-K, the QK reduction and the key bytes read
    (every key row: the H8 screen reads all of a cold block's dimensions)."""

    import torch

    from dsa_amd import _lib, progressive_kernel as P

    block = 64
    nb = C5_LENGTH // block
    items = []
    for v, (keys8, scales) in enumerate(sets):
        per = []
        for b in range(C5_BATCH):
            sel, rem = P.split_head_ids(P.dynamic_head_ids(w[b]).cpu())
            sel, rem = sel.to(device), rem.to(device)
            dgen = torch.Generator().manual_seed(SEED + 131072 + 97 * v + b)
            direct = torch.zeros(nb, dtype=torch.bool)
            direct[torch.randperm(nb, generator=dgen)[: round(PROG_DIRECT_FRACTIONS[32768] * nb)]] = True
            direct = direct.to(device)
            cold = ~direct
            _, maxima = P.h8_block_max_hip(q[b], w[b], keys8[b], sel, cold, block_size=block, key_scales=scales[b])
            values = maxima[cold].cpu()
            promoted = max(1, round(0.10 * values.numel()))
            thr = float(torch.kthvalue(values, max(1, values.numel() - promoted + 1)).values)
            per.append({"sel": sel, "rem": rem, "direct": direct.to(torch.uint8),
                        "thr": torch.tensor([thr], device=device), "cold": cold})
        items.append(per)
    out = torch.empty(C5_BATCH, C5_LENGTH, device=device)
    acc = torch.empty(C5_BATCH, nb, device=device, dtype=torch.int8)
    bmax = torch.empty(C5_BATCH, nb, device=device)
    counter = torch.zeros(C5_BATCH, device=device, dtype=torch.int32)
    top = torch.empty(C5_BATCH, TOPK, device=device, dtype=torch.int64)
    ws = torch.zeros(int(_lib.query("dsa_score_topk_workspace_bytes", C5_BATCH, C5_LENGTH)), device=device,
                     dtype=torch.uint8)
    stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    # The four sequences' inputs packed for one batched launch.
    packed = []
    for per in items:
        packed.append({
            "sel": torch.stack([it["sel"] for it in per]).contiguous(),
            "rem": torch.stack([it["rem"] for it in per]).contiguous(),
            "direct": torch.stack([it["direct"] for it in per]).contiguous(),
            "thr": torch.cat([it["thr"] for it in per]).contiguous(),
        })

    def step(i):
        keys8, scales = sets[i]
        pk = packed[i]
        _lib.call("dsa_progressive_scores_batched", q.data_ptr(), w.data_ptr(), keys8.data_ptr(), scales.data_ptr(),
                  pk["sel"].data_ptr(), pk["rem"].data_ptr(), pk["direct"].data_ptr(), pk["thr"].data_ptr(),
                  out.data_ptr(), None, acc.data_ptr(), bmax.data_ptr(), counter.data_ptr(), C5_BATCH, C5_LENGTH,
                  block, 0, _lib.DTYPE_FP8_E4M3, stream())
        _lib.call("dsa_topk_distributed", out.data_ptr(), C5_BATCH, C5_LENGTH, TOPK, top.data_ptr(), None,
                  ws.data_ptr(), ws.numel(), stream())

    ms = graph_times(step, len(sets), flush, 10, 100, device)
    # Quality of the last key set: recall against the dense step on the same keys.
    from dsa_amd import decode

    keys8, scales = sets[-1]
    dense = decode.indexer_topk(q, w, keys8, TOPK, key_scales=scales)
    step(len(sets) - 1)
    torch.cuda.synchronize()
    recall, qk = [], []
    for b in range(C5_BATCH):
        recall.append(float(torch.isin(dense[b], top[b]).float().mean()))
        direct_count = int(items[-1][b]["direct"].sum())
        promoted_count = int((acc[b].bool() & items[-1][b]["cold"]).sum())
        qk.append(P.progressive_qk_reduction(C5_LENGTH, direct_count, promoted_count, block_size=block))
    st = time_stats(ms)
    return {
        "method": "fused progressive block 64 (fp8), one batched launch over the 4 sequences, + distributed top-2048 "
                  "(3 launches)",
        "step": st,
        "g_keys_per_s": round(C5_BATCH * C5_LENGTH / (st["median_us"] * 1e-6) / 1e9, 3),
        "recall_vs_dense": round(sum(recall) / len(recall), 5),
        "qk_reduction": round(sum(qk) / len(qk), 4),
        "key_bytes_skipped": 0.0,
        "direct_fraction": PROG_DIRECT_FRACTIONS[32768],
        "promotion_target": 0.10,
    }


# --------------------------------------------------------------------------
# The reference's progressive method comparison (benchmark_progressive_dsa.py)
# --------------------------------------------------------------------------
PROG_CONTEXTS = (8192, 16384, 32768)
PROG_DIRECT_FRACTIONS = {8192: 0.945519, 16384: 0.703342, 32768: 0.594227}  # benchmark_progressive_dsa.py:31
PROG_BLOCK = 64
PROG_RATE = 0.10
PROG_VARIANTS = 3


def run_progressive(args) -> None:
    """The reference's method table (benchmark_progressive_dsa.py:300-376) at
    its primary point (block 64, promotion target 0.10, K=2048) for contexts
    8K/16K/32K, one sequence, three synthetic variants rotated: keys ~ N(0,1)
    bf16 with 1% hot keys x4, q ~ N(0,1)/sqrt(128), w ~ N(0,1/64); direct
    blocks drawn as the reference's direct_mask, the promotion threshold as its
    threshold_for_rate (:74-91).  Each method is :124-171's launches with
    torch.topk replaced by the library's exact top-k, timed over 500 calls
    after 50 warm-up, with a 512 MiB flush before each start event."""

    import torch

    from dsa_amd import _lib, metrics as M, progressive_kernel as P

    _lib.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    flush = make_flush(args, device)
    stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    rows = []
    quality = []
    for ctx in PROG_CONTEXTS:
        gen = torch.Generator().manual_seed(SEED + ctx)
        items = []
        for v in range(PROG_VARIANTS):
            q = (torch.randn(64, 128, generator=gen) / math.sqrt(128)).to(torch.bfloat16).to(device)
            w = (torch.randn(64, generator=gen) / 8.0).to(device)
            k = torch.randn(ctx, 128, generator=gen)
            k[torch.randperm(ctx, generator=gen)[: round(HOT_FRACTION * ctx)]] *= 4.0
            k = k.to(torch.bfloat16).to(device)
            blocks = math.ceil(ctx / PROG_BLOCK)
            selected, remaining = P.split_head_ids(P.dynamic_head_ids(w).cpu())
            selected, remaining = selected.to(device), remaining.to(device)
            dgen = torch.Generator(device="cpu").manual_seed(SEED + ctx + PROG_BLOCK + v)
            direct = torch.zeros(blocks, dtype=torch.bool)
            direct[torch.randperm(blocks, generator=dgen)[: round(PROG_DIRECT_FRACTIONS[ctx] * blocks)]] = True
            direct = direct.to(device)
            cold = ~direct
            _, maxima = P.h8_block_max_hip(q, w, k, selected, cold, block_size=PROG_BLOCK)
            values = maxima[cold]
            promoted = max(1, round(PROG_RATE * values.numel()))
            threshold = float(torch.kthvalue(values.cpu(), max(1, values.numel() - promoted + 1)).values) if values.numel() else math.inf
            thr = torch.tensor([threshold], device=device, dtype=torch.float32)
            probe = P.progressive_scores_hip(q, w, k, selected, direct, thr, block_size=PROG_BLOCK, remaining_heads=remaining)
            accepted = int(probe.accepted_blocks.sum().item())
            item = {
                "q": q, "w": w, "k": k, "sel": selected, "rem": remaining, "direct": direct.to(torch.uint8),
                "cold": cold.to(torch.uint8), "all_cold": torch.ones(blocks, dtype=torch.uint8, device=device),
                "thr": thr, "blocks": blocks,
                "full": torch.empty(ctx, device=device), "h8": torch.empty(ctx, device=device),
                "masked": torch.empty(ctx, device=device), "two": torch.empty(ctx, device=device),
                "fused": torch.empty(ctx, device=device), "compact": torch.empty(ctx, device=device),
                "cidx": torch.empty(ctx, device=device, dtype=torch.int32),
                "maxima": torch.empty(blocks, device=device), "keep": torch.empty(blocks, device=device, dtype=torch.uint8),
                "acc": torch.empty(blocks, device=device, dtype=torch.int8), "bmax": torch.empty(blocks, device=device),
                "counter": torch.zeros(1, device=device, dtype=torch.int32),
                "topi": torch.empty(TOPK, device=device, dtype=torch.int64),
                "cand": min(ctx, accepted * PROG_BLOCK), "direct_count": int(direct.sum()),
                "promoted": int((probe.accepted_blocks.bool() & cold).sum()),
                "dscores": torch.empty(1, ctx, device=device),
                "ws": torch.zeros(int(_lib.query("dsa_score_topk_workspace_bytes", 1, ctx)), device=device, dtype=torch.uint8),
            }
            items.append(item)
            # correctness row (benchmark_progressive_dsa.py:230-273)
            full = P.full_scores_hip(q, w, k)
            two = P.two_pass_scores_hip(q, w, k, selected, direct, thr, block_size=PROG_BLOCK)
            keep = probe.accepted_blocks.bool().repeat_interleave(PROG_BLOCK)[:ctx]
            err = (probe.scores[keep] - full[keep]).abs()
            f_ids = M.topk(probe.scores, TOPK, sorted=False)
            t_ids = M.topk(full, TOPK, sorted=False)
            quality.append({"context": ctx, "variant": v, "threshold": threshold, "direct_blocks": item["direct_count"],
                            "promoted_cold_blocks": item["promoted"], "candidate_count": item["cand"],
                            "max_abs_full_error": float(err.max()) if err.numel() else 0.0,
                            "two_fused_max_abs": float(torch.nan_to_num(two.scores - probe.scores).abs().max()),
                            "topk_recall": float(torch.isin(t_ids, f_ids).float().mean()),
                            "qk_reduction": P.progressive_qk_reduction(ctx, item["direct_count"], item["promoted"],
                                                                        block_size=PROG_BLOCK)})

        def full_kernel(it):
            _lib.call("dsa_full_scores", it["q"].data_ptr(), it["w"].data_ptr(), it["k"].data_ptr(), None,
                      it["full"].data_ptr(), 1, ctx, _lib.DTYPE_BF16, stream())

        def h8(it, mask, out):
            _lib.call("dsa_h8_block_max", it["q"].data_ptr(), it["w"].data_ptr(), it["k"].data_ptr(), None, it["sel"].data_ptr(),
                      mask.data_ptr(), out.data_ptr(), it["maxima"].data_ptr(), ctx, PROG_BLOCK, _lib.DTYPE_BF16, stream())

        def masked(it, mask, out):
            _lib.call("dsa_masked_full_scores", it["q"].data_ptr(), it["w"].data_ptr(), it["k"].data_ptr(), None, mask.data_ptr(),
                      out.data_ptr(), ctx, PROG_BLOCK, _lib.DTYPE_BF16, stream())

        def two_pass(it):
            h8(it, it["cold"], it["h8"])
            _lib.call("dsa_promote_blocks", it["direct"].data_ptr(), it["maxima"].data_ptr(), it["thr"].data_ptr(),
                      it["keep"].data_ptr(), it["blocks"], stream())
            masked(it, it["keep"], it["two"])

        def fused(it, compact):
            out = it["compact"] if compact else it["fused"]
            _lib.call("dsa_progressive_scores", it["q"].data_ptr(), it["w"].data_ptr(), it["k"].data_ptr(), None, it["sel"].data_ptr(),
                      it["rem"].data_ptr(), it["direct"].data_ptr(), it["thr"].data_ptr(), out.data_ptr(),
                      it["cidx"].data_ptr() if compact else None, it["acc"].data_ptr(), it["bmax"].data_ptr(),
                      it["counter"].data_ptr(), ctx, PROG_BLOCK, int(compact), _lib.DTYPE_BF16, stream())

        def topk(it, scores, n):
            # the library's choice for one row (metrics.topk): the distributed
            # select from 16K entries, one workgroup below
            if n >= M.DISTRIBUTED_MIN_LENGTH:
                _lib.call("dsa_topk_distributed", scores.data_ptr(), 1, n, min(TOPK, n), it["topi"].data_ptr(), None,
                          it["ws"].data_ptr(), it["ws"].numel(), stream())
            else:
                _lib.call("dsa_topk", scores.data_ptr(), None, 1, n, n, None, min(TOPK, n), 0, it["topi"].data_ptr(), None,
                          stream())

        def decode_step(it):
            _lib.call("dsa_score_topk", it["q"].data_ptr(), it["w"].data_ptr(), it["k"].data_ptr(), None,
                      it["dscores"].data_ptr(), 1, ctx, TOPK, _lib.DTYPE_BF16, it["topi"].data_ptr(), None,
                      it["ws"].data_ptr(), it["ws"].numel(), stream())

        def compact_step(it):
            it["counter"].zero_()  # a fill kernel, not a memset: safe inside a graph
            fused(it, True)
            topk(it, it["compact"], it["cand"])

        methods = {
            "full_kernel": (full_kernel, 1, "kernel"),
            "two_pass_kernel": (two_pass, 3, "kernel"),
            "fused_dense_kernel": (lambda it: fused(it, False), 1, "kernel"),
            "full_plus_topk": (decode_step, 3, "indexer_topk"),
            "temporal_plus_topk": (lambda it: (masked(it, it["direct"], it["masked"]), topk(it, it["masked"], ctx)), 2, "indexer_topk"),
            "h8_plus_topk": (lambda it: (h8(it, it["all_cold"], it["h8"]), topk(it, it["h8"], ctx)), 2, "indexer_topk"),
            "two_pass_plus_topk": (lambda it: (two_pass(it), topk(it, it["two"], ctx)), 4, "indexer_topk"),
            "fused_dense_plus_topk": (lambda it: (fused(it, False), topk(it, it["fused"], ctx)), 2, "indexer_topk"),
            "fused_compact_plus_topk": (compact_step, 3, "indexer_topk"),
        }
        for name, (fn, launches, scope) in methods.items():
            ms = graph_times(lambda i, fn=fn: fn(items[i]), PROG_VARIANTS, flush, 50, 500, device)
            row = {"context": ctx, "method": name, "scope": scope, "block_size": PROG_BLOCK, "promotion_target": PROG_RATE,
                   "topk": TOPK, "kernel_launches": launches, **time_stats(ms)}
            rows.append(row)
            print(json.dumps(row), file=sys.stderr, flush=True)
        del items
        torch.cuda.empty_cache()
    full32 = next(r for r in rows if r["context"] == 32768 and r["method"] == "full_plus_topk")
    line = {
        "metric": "reference method table on MI355X: full / H8 / two-pass / fused progressive (+ exact top-K2048), one sequence, 8K/16K/32K",
        "value": round(32768 / (full32["median_us"] * 1e-6) / 1e9, 3),
        "unit": "G keys/s (full + top-K at 32K, median)",
        "n_gpus": 1,
        "steps": 500,
        "warmup": 50,
        "ms_per_step": round(full32["median_us"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "benchmark_progressive_dsa.py primary point: block 64, promotion 0.10, K=2048, "
                   f"direct fractions 0.946/0.703/0.594, 3 synthetic variants rotated, 512 MiB {args.flush} flush"},
        "rows": len(rows),
        "quality": quality,
    }
    write_table(args, line, rows)
    print(json.dumps(line), flush=True)





# --------------------------------------------------------------------------
# Sidecar encoders: the producers of the indexer's q, w and K
# --------------------------------------------------------------------------
SIDECAR_HIDDEN = 2048


def torch_formula_encode(module, hidden, positions, cache, rows):
    """Baseline: the reference's encoder formula (sidecar.py:10-88) as torch
    eager ops on the same GPU and weights -- projection, LayerNorm, the
    non-interleaved RoPE by slices, products and a concatenation -- then the
    key-cache append by index_copy_."""

    import torch
    from torch.nn import functional as F

    def rope(x, pos):
        half = module.rope_dim // 2
        inv = module.rope_theta ** (-torch.arange(half, device=x.device, dtype=torch.float32) / half)
        ang = pos.to(torch.float32).unsqueeze(-1) * inv
        cos, sin = torch.cos(ang).to(x.dtype), torch.sin(ang).to(x.dtype)
        while cos.ndim < x.ndim:
            cos, sin = cos.unsqueeze(-2), sin.unsqueeze(-2)
        a, b = x[..., :half], x[..., half:]
        return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)

    def partial(x, pos):
        return torch.cat((rope(x[..., : module.rope_dim], pos), x[..., module.rope_dim:]), dim=-1)

    keys = partial(F.layer_norm(F.linear(hidden, module.wk.weight), (module.head_dim,), module.k_norm.weight,
                                module.k_norm.bias, module.k_norm.eps), positions)
    cache.index_copy_(0, rows, keys.reshape(-1, module.head_dim))
    q = F.linear(hidden, module.wq.weight).view(*hidden.shape[:-1], module.heads, module.head_dim)
    q = partial(q, positions)
    w = F.linear(hidden.float(), module.weights_proj.weight.float()) * (module.heads * module.head_dim) ** -0.5
    return q, w


def run_sidecar(args) -> None:
    """The indexer sidecar's encoders (reference sidecar.py:31-88, bf16 module,
    hidden 2048, 64 heads x 128 dims, rope_dim 64) per decode step (16
    sequences, one new token each, keys appended to a 16 x 32768-row cache)
    and per prefill chunk (4096 tokens).  Reports the library path (platform
    GEMMs + the fused HIP epilogues) and the reference formula as torch eager
    ops on the same GPU, HIP events around each call after a cache flush,
    median over 100."""

    import torch
    from torch.nn import functional as F

    from dsa_amd import _lib, sidecar

    _lib.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    torch.manual_seed(SEED)
    module = sidecar.LightningIndexerSidecar(hidden_size=SIDECAR_HIDDEN).to(device=device, dtype=torch.bfloat16)
    module.eval()
    flush = make_flush(args, device)
    results = {}
    for name, tokens in (("decode", BATCH), ("prefill", 4096)):
        hidden = torch.randn(tokens, SIDECAR_HIDDEN, device=device, dtype=torch.bfloat16)
        positions = torch.randint(0, LENGTH, (tokens,), device=device)
        cache = torch.zeros(BATCH * LENGTH, 128, device=device, dtype=torch.bfloat16)
        rows = torch.randperm(BATCH * LENGTH, device=device)[:tokens]

        def library():
            module.encode_keys(hidden, positions, out=cache, out_rows=rows)
            return module.encode_queries(hidden, positions)

        def formula():
            return torch_formula_encode(module, hidden, positions, cache, rows)

        def epilogues_only():
            # the HIP pass alone, on precomputed projections
            _lib.call("dsa_encode_keys_epilogue", _lib.ptr(pk), _lib.DTYPE_BF16, 128, _lib.ptr(lw), _lib.ptr(lb),
                      1e-6, _lib.ptr(positions), 64, 10_000.0, _lib.ptr(cache), _lib.DTYPE_BF16, 128, _lib.ptr(rows),
                      cache.shape[0], tokens, 128, torch.cuda.current_stream().cuda_stream)
            _lib.call("dsa_encode_queries_epilogue", _lib.ptr(pq), _lib.ptr(pw), _lib.ptr(positions), 64, 10_000.0,
                      float((64 * 128) ** -0.5), _lib.ptr(oq), _lib.ptr(ow), tokens, 64, 128, _lib.DTYPE_BF16,
                      torch.cuda.current_stream().cuda_stream)

        with torch.no_grad():
            pk = F.linear(hidden, module.wk.weight).contiguous()
            pq = F.linear(hidden, module.wq.weight).contiguous()
            pw = F.linear(hidden.float(), module.weights_proj.weight.float()).contiguous()
            lw = module.k_norm.weight.float().contiguous()
            lb = module.k_norm.bias.float().contiguous()
            oq = torch.empty_like(pq)
            ow = torch.empty_like(pw)
            q_lib, w_lib = library()
            q_ref, w_ref = formula()
            q_diff = float((q_lib.float() - q_ref.float()).abs().max())
            w_diff = float((w_lib - w_ref).abs().max())
            timings = {}
            for label, fn in (("library", library), ("torch_formula", formula), ("epilogues", epilogues_only)):
                ms = []
                for it in range(110):
                    flush()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    fn()
                    e1.record()
                    torch.cuda.synchronize()
                    if it >= 10:
                        ms.append(e0.elapsed_time(e1))
                timings[label] = time_stats(ms)
            # The same calls captured in a HIP graph and replayed: GPU time
            # without the host's per-launch cost (one sequence of launches per
            # replay, a cache flush before each).
            for label, fn in (("library", library), ("torch_formula", formula)):
                graph = torch.cuda.CUDAGraph()
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    fn()  # warm the allocator on the capture stream
                torch.cuda.current_stream().wait_stream(side)
                with torch.cuda.graph(graph):
                    fn()
                ms = []
                for it in range(60):
                    flush()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    graph.replay()
                    e1.record()
                    torch.cuda.synchronize()
                    if it >= 10:
                        ms.append(e0.elapsed_time(e1))
                timings[f"{label}_graph"] = time_stats(ms)
                del graph
        weight_bytes = (module.wq.weight.numel() + module.wk.weight.numel()) * 2 + module.weights_proj.weight.numel() * 4
        epi_bytes = tokens * (128 * 2 * 2 + 64 * 128 * 2 * 2 + 64 * 4 * 2 + 8 + 8)
        results[name] = {
            "tokens": tokens,
            **{f"{k}_us": v["median_us"] for k, v in timings.items()},
            "speedup_vs_torch_formula": round(timings["torch_formula"]["median_us"] / timings["library"]["median_us"], 3),
            "weight_bytes": weight_bytes,
            "weight_stream_floor_us": round(weight_bytes / HBM_PEAK_GBS / 1e3, 3),
            "epilogue_bytes": epi_bytes,
            "epilogue_gbs": round(epi_bytes / (timings["epilogues"]["median_us"] * 1e-6) / 1e9, 1),
            "max_abs_diff_vs_formula": {"queries": q_diff, "weights": w_diff},
            "timings": timings,
        }
    dec = results["decode"]
    line = {
        "metric": "sidecar encoders: us per decode step (16 tokens: keys appended to the cache, queries + head weights)",
        "value": dec["library_us"],
        "unit": "us",
        "n_gpus": 1,
        "steps": 100,
        "warmup": 10,
        "ms_per_step": round(dec["library_us"] / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "LightningIndexerSidecar(hidden 2048, 64 x 128, rope_dim 64), bf16, random init; "
                   "decode: 16 tokens, prefill: 4096 tokens"},
        "roofline": {"bound": "hbm", "achieved": round(dec["weight_bytes"] / (dec["library_us"] * 1e-6) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dec["weight_bytes"] / (dec["library_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": "decode step: weight streaming of wq/wk/weights_proj + epilogues",
                     "algorithmic_bytes": dec["weight_bytes"]},
        "shapes": results,
        "timing": f"HIP events around each call, 512 MiB {args.flush} flush before each, median over 100",
    }
    write_table(args, line, [])
    print(json.dumps(line), flush=True)



# --------------------------------------------------------------------------
# Two-path verifier (live decode step) at the C3 shape
# --------------------------------------------------------------------------
VERIFIER_STEPS = 32
VERIFIER_GAMMA_SIGMA = (-0.25, -0.5, -1.0)  # margins of the temporal policy, in units of the score std
VERIFIER_HEADLINE_GAMMA = -0.5
VERIFIER_CONFIGS = (
    # name, path, width, rescue fraction, dims strategy, bits
    ("head_dynamic_abs_w8_b64_r0.1", "head", 8, 0.1, None, None),
    ("head_dynamic_abs_w16_b64_r0.1", "head", 16, 0.1, None, None),
    ("dim_had_even_w16_b64_r0.1", "dim", 16, 0.1, "even", None),
    ("dim_had_random_w32_int4_b64_r0.1", "dim", 32, 0.1, "random", 4),
)


def run_verifier(args) -> None:
    """The live verifier step (reference verifier.py:173-392 as a decode
    step) on the C3 shape: B=4 sequences from 16384 keys, one key appended per
    step, K=2048, block 64, the reference's selected two-path configs
    (configs/two_path_full_selected.json: head width 8 / 16 with dynamic
    |w| routing, dim width 16 even / 32 random with a Hadamard rotation) over a
    dynamic previous-max own-trajectory policy at three margins, beside the
    temporal step alone and the dense step
    (scores + exact top-k).  HIP events around each step (eager, every launch
    included), median over the steps; recall and byte accounting from the
    reference's metrics dict against the dense step of the same inputs."""

    import numpy as np
    import torch

    from dsa_amd import _lib, approx, decode, verifier, verifier_scoring

    _lib.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    keys, w, queries = c3_inputs(device)
    steps = min(VERIFIER_STEPS, len(queries) - 1)
    k, block = C3_TOPK, 64
    start = C3_LENGTH
    flush = make_flush(args, device)

    def timed(fn):
        flush()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        out = fn()
        e1.record()
        torch.cuda.synchronize()
        return out, e0.elapsed_time(e1)

    # the dense step of every decode step: truth for the metrics, and the baseline timing
    dense_rows, dense_ms = [], []
    for t in range(steps + 1):
        cur = start + t
        kv = keys[:, :cur].contiguous()
        (idx, sc), ms = timed(lambda: decode.indexer_topk(queries[t], w, kv, k, return_scores=True))
        dense_rows.append(sc)
        if t:
            dense_ms.append(ms)
    sigma = float(dense_rows[0].std())
    blocks = -(-(start + steps) // block)
    wave = c3_wave(blocks, block, args.c3_refreshes)
    rows = []
    summary = {}
    for gamma_sigma in VERIFIER_GAMMA_SIGMA:
        policy = approx.ApproxPolicy(name="dynamic_previous_max", gamma=gamma_sigma * sigma, cold_streak=0,
                                     dynamic_threshold=True, order="previous_max")
        runs = [("temporal_only", None, 0, 0.0, None, None), *VERIFIER_CONFIGS]
        for name, path, width, fraction, strategy, bits in runs:
            state = approx.initialize_state(dense_rows[0], k=k, block_size=block, capacity=start + steps)
            cfg = None
            kwargs = {}
            if path is not None:
                cfg = verifier.VerifierConfig(
                    name=name, path=path, width=width, score_ratio=width / 64 if path == "head" else width / 128,
                    block_size=block, rescue_fraction=fraction,
                    sketch_bytes_per_token=0.0 if path == "head" else width * (bits or 16) / 8)
            if path == "dim":
                dims = (np.linspace(0, 127, width).astype(np.int64) if strategy == "even"
                        else np.sort(np.random.default_rng(SEED).choice(128, width, replace=False)))
                scale = None
                if bits is not None:
                    scale = verifier._tensor_scale(verifier.dim_sketch(keys, dims), bits)
                kwargs["key_sketch"] = verifier.sketch_keys(keys, dims, bits=bits, scale=scale)
                kwargs["sketch_scale"] = scale
            ms_all, metric_rows, recalls = [], [], []
            for t in range(1, steps + 1):
                cur = start + t
                if path is None:
                    out, ms = timed(lambda: approx.approx_step(state, queries[t], w, keys[:, :cur], policy=policy,
                                                               step=t, wave=wave))
                    ms_all.append(ms)
                    truth = decode.indexer_topk(queries[t], w, keys[:, :cur].contiguous(), k)
                    for b in range(C3_BATCH):
                        recalls.append(np.intersect1d(out.topk[b].cpu().numpy(), truth[b].cpu().numpy()).size / k)
                    continue
                if path == "head":
                    kwargs["head_ids"] = verifier_scoring.dynamic_head_indices(w, width, "high_weight")
                else:
                    kwargs["query_sketch"] = verifier.sketch_queries(queries[t], dims, bits=bits, scale=scale)
                out, ms = timed(lambda: verifier.verifier_step(state, queries[t], w, keys[:, :cur], policy=policy,
                                                               config=cfg, step=t, wave=wave, **kwargs))
                ms_all.append(ms)
                for b in range(C3_BATCH):
                    metric_rows.append(verifier.verifier_metrics(out, dense_rows[t], config=cfg, policy=policy,
                                                                 step=t, row=b))
            key = f"{name}@gamma{gamma_sigma}"
            if path is None:
                summary[key] = {"us_per_step": time_stats(ms_all)["median_us"],
                                "recall_mean": round(float(np.mean(recalls)), 5)}
                continue
            col = lambda f: np.asarray([r[f] for r in metric_rows], dtype=np.float64)  # noqa: E731
            summary[key] = {
                "us_per_step": time_stats(ms_all)["median_us"],
                "recall_mean": round(float(col("recall").mean()), 5),
                "exact_match": round(float(col("exact_match").mean()), 4),
                "net_qk_reduction_median": round(float(np.median(col("net_qk_reduction"))), 4),
                "ideal_key_byte_reduction_median": round(float(np.median(col("ideal_key_byte_reduction"))), 4),
                "physical_b64_key_byte_reduction_median": round(
                    float(np.median(col("physical_b64_key_byte_reduction"))), 4),
                "cold_tokens_scanned_median": float(np.median(col("cold_tokens_scanned"))),
                "rescue_blocks_median": float(np.median(col("rescue_blocks"))),
                "newly_active_block_recall": round(float(col("newly_active_block_recall").mean()), 4),
            }
            rows.extend({"verifier": name, "gamma_sigma": gamma_sigma, **r} for r in metric_rows)
    dense_us = time_stats(dense_ms)["median_us"]
    head = summary[f"{VERIFIER_CONFIGS[0][0]}@gamma{VERIFIER_HEADLINE_GAMMA}"]
    line = {
        "metric": "two-path verifier decode step: us per step (B=4, L=16K+, K=2048, block 64) and Recall@K vs dense",
        "value": head["us_per_step"],
        "unit": "us",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 0,
        "ms_per_step": round(head["us_per_step"] / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"C3 shape: B={C3_BATCH}, L={start}+t, K={k}, block {block}, dynamic previous-max "
                   f"own-trajectory policy, gamma {VERIFIER_GAMMA_SIGMA} sigma (headline {VERIFIER_HEADLINE_GAMMA}), "
                   f"threshold refresh every {wave} blocks, {steps} decode steps",
                   "verifiers": [c[0] for c in VERIFIER_CONFIGS]},
        "dense_step_us": dense_us,
        "verifiers": summary,
        "timing": f"HIP events around each eager step, 512 MiB {args.flush} flush before each, median over the steps",
    }
    write_table(args, line, rows)
    print(json.dumps(line), flush=True)



# --------------------------------------------------------------------------
# Trace replay (the reference's analysis sweep) on a GPU-collected trace
# --------------------------------------------------------------------------
REPLAY_STEPS = 9
REPLAY_K = (2048,)
REPLAY_GAMMAS = (0.0, 0.25, 0.5, 1.0)


def run_replay(args) -> None:
    """The reference's replay_trace sweep (replay.py:476-627; configs/pilot.yaml:
    K=2048, blocks 16/32/64/128, gamma_sigma 0/0.25/0.5/1, every method and
    order, threshold refreshed after every block as the reference does) over a
    dense score trace of one sequence collected on the GPU (C3 shape: 16384
    keys + one per step, AR(1) queries rho=0.95, N(0,1) bf16 keys).  Reports
    transitions per second of the GPU replay (every filter in the HIP temporal
    kernels) and of the CPU restatement of the reference's replay on a
    bounded sample of the same transitions."""

    import numpy as np
    import torch

    from dsa_amd import _lib, replay
    from dsa_amd.trace import collect_trace

    _lib.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    gen = torch.Generator().manual_seed(SEED)
    steps = REPLAY_STEPS
    keys = torch.randn(C3_LENGTH + steps - 1, 128, generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn(64, generator=gen) / 8.0).to(device)
    q = torch.randn(64, 128, generator=gen) / math.sqrt(128)
    qs = []
    for _ in range(steps):
        qs.append(q.to(torch.bfloat16))
        q = C3_RHO * q + math.sqrt(1 - C3_RHO * C3_RHO) * torch.randn(64, 128, generator=gen) / math.sqrt(128)
    trace = collect_trace(torch.stack(qs).to(device), w, keys, np.arange(C3_LENGTH, C3_LENGTH + steps))
    kwargs = dict(k_values=list(REPLAY_K), block_sizes=list(C3_BLOCKS), gamma_sigma_values=list(REPLAY_GAMMAS))
    # warm the workspaces and kernels on the first transition
    first = type(trace)(trace.scores[:2], trace.lengths[:2], 0, "synthetic", "0", {})
    replay.replay_trace_rows(first, **kwargs)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    rows = replay.replay_trace_rows(trace, **kwargs)
    torch.cuda.synchronize()
    gpu_s = time.perf_counter() - t0
    transitions = steps - 1
    per_transition = len(rows) // transitions
    summary = replay.aggregate_rows(__import__("pandas").DataFrame(rows))
    best = summary[summary.recall >= 0.999].sort_values("net_byte_reduction", ascending=False).head(1).to_dict("records")
    cpu = None
    if not args.no_cpu_baseline:
        import os

        from oracle import replay as R

        rows_h = [trace.row(0), trace.row(1)]
        c0 = time.perf_counter()
        sample_rows = R.replay_trace_rows(rows_h, **kwargs)
        cpu_s = time.perf_counter() - c0
        cpu = {"value": round(len(sample_rows) / cpu_s, 2), "unit": "replay rows/s", "cores": 1, "kind": "port",
               "sample": f"the {len(sample_rows)} rows of the trace's first transition (the same sweep) in "
                         f"{cpu_s:.1f} s on 1 of {os.cpu_count()} host threads (oracle/replay.py, the reference's "
                         "replay restated)"}
    line = {
        "metric": "trace replay: replay rows per second (the reference's replay_trace sweep, C3-shape trace)",
        "value": round(len(rows) / gpu_s, 2),
        "unit": "replay rows/s",
        "n_gpus": 1,
        "steps": transitions,
        "warmup": 1,
        "ms_per_step": round(gpu_s / transitions * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": f"replay_trace over a GPU-collected trace: L {C3_LENGTH}+t, {transitions} transitions, "
                   f"K {list(REPLAY_K)}, blocks {list(C3_BLOCKS)}, gamma_sigma {list(REPLAY_GAMMAS)}, "
                   f"{per_transition} rows per transition, wave 1"},
        "gpu_seconds": round(gpu_s, 3),
        "rows": len(rows),
        "best_at_recall_0.999": best[0] if best else None,
        "cpu_baseline": cpu,
    }
    write_table(args, line, rows)
    print(json.dumps(line, default=float), flush=True)


if __name__ == "__main__":
    main()
