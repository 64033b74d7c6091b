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
    assert lib.dsa_masked_full_scores(fake, fake, fake, fake, fake, 64, 48, 2, None) == 1
    assert b"block_size" in lib.dsa_last_error()
    # unsupported dtype
    assert lib.dsa_score_queries(fake, 8192, fake, 64, None, 0, 64, fake, 16, 1, None, 0, fake, 16, 1, 16, -1, 0, None) == 1
    assert lib.dsa_topk_long_workspace_bytes(2, 100000, 2048) == 2 * 4 * 2048 * 12


def test_call_raises_runtime_error_with_message() -> None:
    with pytest.raises(RuntimeError, match="dsa_topk failed"):
        _lib.call("dsa_topk", None, None, 1, 16, 16, None, 4, 1, None, None, None)
