"""The trace format (reference trace.py:11-62): ScoreTrace checks, and the
.npz round trip through save_trace / load_trace, including the reference's
metadata layout (a JSON string with layer, workload and prompt id)."""

from __future__ import annotations

import json

import numpy as np
import pytest

from dsa_amd.cli import build_parser
from dsa_amd.trace import ScoreTrace, load_trace, save_trace


def _trace() -> ScoreTrace:
    scores = np.full((3, 6), -np.inf, dtype=np.float16)
    lengths = np.array([4, 5, 6])
    for t, n in enumerate(lengths):
        scores[t, :n] = np.arange(n) + t
    return ScoreTrace(scores=scores, lengths=lengths, layer=7, workload="w", prompt_id="p1", metadata={"rho": 0.9})


def test_trace_checks_and_rows() -> None:
    trace = _trace()
    np.testing.assert_array_equal(trace.row(1), np.arange(5, dtype=np.float32) + 1)
    assert trace.row(2).dtype == np.float32
    with pytest.raises(ValueError):
        ScoreTrace(np.zeros(3), np.array([1]), 0, "w", "p", {})
    with pytest.raises(ValueError):
        ScoreTrace(np.zeros((2, 3)), np.array([1]), 0, "w", "p", {})
    with pytest.raises(ValueError):
        ScoreTrace(np.zeros((2, 3)), np.array([1, 4]), 0, "w", "p", {})


def test_save_load_round_trip(tmp_path) -> None:
    trace = _trace()
    path = tmp_path / "sub" / "t.npz"
    save_trace(path, trace)
    with np.load(path, allow_pickle=False) as data:
        meta = json.loads(str(data["metadata"].item()))
        assert meta == {"layer": 7, "workload": "w", "prompt_id": "p1", "rho": 0.9}
        assert data["scores"].dtype == np.float16
    back = load_trace(path)
    np.testing.assert_array_equal(back.scores, trace.scores)
    np.testing.assert_array_equal(back.lengths, trace.lengths)
    assert (back.layer, back.workload, back.prompt_id, back.metadata) == (7, "w", "p1", {"rho": 0.9})


def test_cli_parses_reference_arguments(tmp_path) -> None:
    args = build_parser().parse_args(["analyze", "--trace-roots", str(tmp_path), "--output", str(tmp_path / "o"),
                                      "--wave", "4"])
    assert args.command == "analyze" and args.wave == 4 and args.trace_roots == [tmp_path]
    args = build_parser().parse_args(["collect", "--output", str(tmp_path / "t.npz"), "--steps", "3"])
    assert args.steps == 3 and args.length == 16384
