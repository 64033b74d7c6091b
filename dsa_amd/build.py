"""Build recipe for libdsa_amd.so (gfx950 only).

Every ``csrc/*.hip`` and ``csrc/*.cpp`` file is compiled by ``hipcc`` into an
object under ``dsa_amd/_build/`` and linked into ``dsa_amd/libdsa_amd.so``,
which is loaded with ctypes by :mod:`dsa_amd._lib`.  Run ``python -m
dsa_amd.build`` (or ``__graft_entry__.build()``) after editing a source.

``python -m dsa_amd.build --trace`` builds ``dsa_amd/libdsa_amd_trace.so``
instead: the same kernels compiled with ``-DDSA_PHASE_TRACE``, in which the
decode scoring kernel and the fused static temporal kernel record per-
workgroup phase timestamps (read by :mod:`dsa_amd.phase_trace`).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIBRARY = PACKAGE_DIR / "libdsa_amd.so"
TRACE_BUILD_DIR = PACKAGE_DIR / "_build_trace"
TRACE_LIBRARY = PACKAGE_DIR / "libdsa_amd_trace.so"
INCLUDE_DIR = PACKAGE_DIR.parent / "include"
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled for device code; hipcc's host pass warns
# that it does not know the feature, which is harmless.
COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    candidates = [os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"]
    for candidate in candidates:
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the HIP extension cannot be built")


def _compile(hipcc: str, source: Path, build_dir: Path, extra: list[str]) -> Path:
    obj = build_dir / (source.name + ".o")
    cmd = [hipcc, *COMMON_FLAGS, *extra, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{stderr}")
    if stderr.strip():
        print(stderr, file=sys.stderr)
    return obj


def build(verbose: bool = True, trace: bool = False) -> Path:
    """Compile every source and link the shared library (the phase-trace
    variant with ``trace``); returns its path."""

    hipcc = _hipcc()
    build_dir = TRACE_BUILD_DIR if trace else BUILD_DIR
    library = TRACE_LIBRARY if trace else LIBRARY
    extra = ["-DDSA_PHASE_TRACE"] if trace else []
    build_dir.mkdir(exist_ok=True)
    sources = sorted([*SOURCE_DIR.glob("*.hip"), *SOURCE_DIR.glob("*.cpp")])
    if not sources:
        raise RuntimeError(f"no sources under {SOURCE_DIR}")
    workers = min(len(sources), max(1, (os.cpu_count() or 4) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda src: _compile(hipcc, src, build_dir, extra), sources))
    tmp = library.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, library)
    if verbose:
        print(f"built {library} from {len(sources)} sources", file=sys.stderr)
    return library


if __name__ == "__main__":
    build(trace="--trace" in sys.argv[1:])
