"""The C-ABI library loads, exports every symbol the public header declares,
and rejects invalid arguments before touching a device (CPU-only checks)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from dsa_amd import _lib

HEADER_DIR = Path(__file__).resolve().parents[1] / "include"


def declared_symbols() -> list[str]:
    names = []
    for header in HEADER_DIR.glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"\b(dsa_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_binding_table() -> None:
    assert declared_symbols() == _lib.exported_names()


def test_library_exports_every_declared_symbol() -> None:
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.dsa_abi_version() == _lib.ABI_VERSION


def test_invalid_arguments_are_rejected_without_a_device() -> None:
    lib = _lib.load()
    assert lib.dsa_topk(None, None, 1, 16, 16, None, 4, 1, None, None, None) == 1
    assert b"scores" in lib.dsa_last_error()
    assert lib.dsa_full_scores(None, None, None, None, None, 1, 16, 2, None) == 1
    fake = ctypes.c_void_p(256)
    # bad block size is reported before any launch
    assert lib.dsa_masked_full_scores(fake, fake, fake, None, fake, fake, 64, 48, 2, None) == 1
    assert b"block_size" in lib.dsa_last_error()
    # unsupported dtype
    assert lib.dsa_score_queries(fake, 8192, fake, 64, None, 0, 64, fake, 16, 1, None, 0, fake, 16, 1, 16, -1, 0, None) == 1
    assert lib.dsa_topk_long_workspace_bytes(2, 100000, 2048) == 2 * 4 * 2048 * 12


def test_call_raises_runtime_error_with_message() -> None:
    with pytest.raises(RuntimeError, match="dsa_topk failed"):
        _lib.call("dsa_topk", None, None, 1, 16, 16, None, 4, 1, None, None, None)


def test_approx_policy_struct_matches_the_header() -> None:
    # four doubles, then eight int32 fields, no padding: 64 bytes
    assert ctypes.sizeof(_lib.ApproxPolicyC) == 64
    assert _lib.ApproxPolicyC.risk_model.offset == 32
    assert _lib.ApproxPolicyC.history.offset == 60


def test_approx_step_rejects_bad_policies_without_a_device() -> None:
    lib = _lib.load()
    fake = ctypes.c_void_p(256)
    policy = _lib.ApproxPolicyC(ema_alpha=0.9, risk_model=0, order=2, buckets=0, cold_streak=1, age_cap=-1)
    args = [fake, fake, fake, 4096, None, ctypes.addressof(policy), None, 4096, fake, fake, fake, fake, fake, fake, 64,
            fake, fake, fake, fake, 2, 4096, 512, 64, 1, 2, fake, 1 << 20, None]
    assert lib.dsa_approx_step(*args) == 1
    assert b"bucket" in lib.dsa_last_error()
    policy.order, policy.risk_model = 1, 5
    assert lib.dsa_approx_step(*args) == 1
    assert b"risk_model" in lib.dsa_last_error()
    policy.risk_model = 1
    args[14] = 63  # state rows shorter than the 64 blocks of L=4096 at block 64
    assert lib.dsa_approx_step(*args) == 1
    assert b"state_stride" in lib.dsa_last_error()
