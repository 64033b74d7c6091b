"""ctypes binding of libdsa_amd.so (the C ABI declared in include/dsa_amd.h).

The library is loaded lazily from the package directory.  There is no
fallback: if the shared object is missing or does not load, every GPU entry
point raises ``RuntimeError("HIP extension not built ...")``.
"""

from __future__ import annotations

import atexit
import ctypes
import threading
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libdsa_amd.so"
ABI_VERSION = 5

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_FP8_E4M3 = 3
DTYPE_F64 = 4  # score rows of dsa_topk_exact only

_TORCH_DTYPES = {
    torch.float32: DTYPE_F32,
    torch.float16: DTYPE_F16,
    torch.bfloat16: DTYPE_BF16,
    torch.float8_e4m3fn: DTYPE_FP8_E4M3,
}

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64

# name -> argument types (every entry point returns int32 status unless listed)
_SIGNATURES: dict[str, list] = {
    "dsa_full_scores": [_p, _p, _p, _p, _p, _i64, _i64, _i32, _p],
    "dsa_score_queries": [
        _p, _i64, _p, _i64, _p, _i64, _i32, _p, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64,
        _i64, _i32, _p,
    ],
    "dsa_score_queries_topk": [
        _p, _i64, _p, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p, _p, _i64, _p,
    ],
    "dsa_route_heads": [_p, _i64, _i64, _i64, _i32, _p, _p, _p],
    "dsa_pair_moments": [_p, _p, _i32, _i64, _p, _p, _p],
    "dsa_average_ranks": [_p, _i32, _p, _i64, _p, _p],
    "dsa_index_overlap": [_p, _p, _i64, _p, _p],
    "dsa_block_streaks": [_p, _p, _i64, _p, _p, _p, _p, _p],
    "dsa_score_topk": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p, _p, _p, _i64, _p],
    "dsa_score_topk_noalloc": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p, _p, _p],
    "dsa_score_hist": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p, _i64, _p],
    "dsa_select_topk": [_p, _i64, _i64, _i64, _p, _p, _p, _i64, _p],
    "dsa_score_hist_timed": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p, _i64, _p, _p, _p],
    "dsa_select_topk_timed": [_p, _i64, _i64, _i64, _p, _p, _p, _i64, _p, _p, _p],
    "dsa_topk_distributed": [_p, _i64, _i64, _i64, _p, _p, _p, _i64, _p],
    "dsa_h8_block_max": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _p],
    "dsa_masked_full_scores": [_p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _p],
    "dsa_progressive_scores": [
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _p,
    ],
    "dsa_promote_blocks": [_p, _p, _p, _p, _i64, _p],
    "dsa_progressive_scores_batched": [
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _p,
    ],
    "dsa_topk": [_p, _p, _i64, _i64, _i64, _p, _i64, _i32, _p, _p, _p],
    "dsa_topk_long": [_p, _i64, _i64, _i64, _i32, _p, _p, _p, _i64, _p],
    "dsa_topk_exact": [_p, _i32, _i64, _i64, _i64, _i64, _i32, _p, _p, _p, _i64, _p],
    "dsa_block_max": [_p, _i64, _i64, _i64, _i32, _p, _p],
    "dsa_project_gemm": [_p, _i32, _i64, _i64, _i64, _p, _i32, _i64, _p, _i64, ctypes.c_float, _p, ctypes.c_float,
                         _p, _i64, _p],
    "dsa_rope": [_p, _p, _p, _i64, _i32, _i32, _i32, ctypes.c_float, _i32, _p],
    "dsa_encode_keys_epilogue": [_p, _i32, _i64, _p, _p, ctypes.c_float, _p, _i32, ctypes.c_float, _p, _i32, _i64,
                                 _p, _i64, _i64, _i32, _p],
    "dsa_encode_queries_epilogue": [_p, _p, _p, _i32, ctypes.c_float, ctypes.c_float, _p, _p, _i64, _i32, _i32,
                                    _i32, _p],
    "dsa_block_key_norms": [_p, _i64, _i64, _i64, _i32, _i32, _p, _p],
    "dsa_temporal_score_radius": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p],
    "dsa_temporal_step": [
        _p, _p, _p, _i64, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32,
        _p, _i64, _p,
    ],
    "dsa_temporal_keys_loaded": [_p, _i64, _i64, _i64, _i32, _p, _p],
    "dsa_certified_margins": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _p, _p],
    "dsa_approx_step": [
        _p, _p, _p, _i64, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i64,
        _i32, _i32, _i32, _p, _i64, _p,
    ],
    "dsa_approx_init_state": [_p, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _p],
    "dsa_verifier_step": [
        _p, _p, _p, _i64, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64,  # temporal step and policy state
        _p, _p, _i64, _p, _p, _i64,  # spec, head ids, sketches
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,  # outputs
        _i64, _i64, _i64, _i32, _i32, _i32, _p, _i64, _p,
    ],
    "dsa_temporal_replay_step": [
        _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _p, _i64, _p,
    ],
    "dsa_stream_read": [_p, _i64, _i32, _p, _p, _p, _p],
    "dsa_verifier_replay_step": [
        _p, _i64, _p, _i64, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p,  # rows, policy, state, spec
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,  # outputs
        _i64, _i64, _i64, _i32, _i32, _p, _i64, _p,
    ],
    "dsa_approx_replay_step": [
        _p, _i64, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _p,
        _i64, _p,
    ],
    "dsa_project_rows": [_p, _i64, _i64, _p, _i32, _i64, _i64, _p, _i64, _p],
    "dsa_project_rows_pair": [_p, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p],
    "dsa_dim_sketch": [_p, _i64, _i32, _i32, _p, _i32, _i32, _i32, ctypes.c_float, _p, _i32, _p],
    "dsa_abs_max": [_p, _i64, _i32, _p, _p],
    "dsa_fake_quantize": [_p, _i64, _i32, _i32, ctypes.c_float, _p, _p, _p],
    "dsa_sketch_scores": [_p, _p, _i64, _i32, _p, _i32, ctypes.c_float, _i32, _i64, _p, _p],
}
_RESTYPES: dict[str, object] = {
    "dsa_topk_long_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "dsa_score_topk_workspace_bytes": (_i64, [_i64, _i64]),
    "dsa_temporal_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32]),
    "dsa_topk_exact_workspace_bytes": (_i64, [_i64, _i64, _i32]),
    "dsa_project_gemm_workspace_bytes": (_i64, [_i64]),
}



class ApproxPolicyC(ctypes.Structure):
    """``dsa_approx_policy`` of include/dsa_amd.h."""

    _fields_ = [
        ("gamma", ctypes.c_double),
        ("age_slope", ctypes.c_double),
        ("ema_alpha", ctypes.c_double),
        ("volatility_lambda", ctypes.c_double),
        ("risk_model", _i32),
        ("order", _i32),
        ("buckets", _i32),
        ("cold_streak", _i32),
        ("age_cap", _i32),
        ("recent_window", _i32),
        ("full_refresh", _i32),
        ("history", _i32),
    ]


class VerifierSpecC(ctypes.Structure):
    """``dsa_verifier_spec`` of include/dsa_amd.h."""

    _fields_ = [
        ("path", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("promotion", ctypes.c_int32),
        ("sketch_codes", ctypes.c_int32),
        ("rescue_fraction", ctypes.c_double),
        ("promotion_threshold", ctypes.c_float),
        ("sketch_scale", ctypes.c_float),
    ]


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def exported_names() -> list[str]:
    """Every symbol this binding expects the library to export."""

    return sorted([*_SIGNATURES, *_RESTYPES, "dsa_last_error", "dsa_abi_version"])


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is not built."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY_PATH.exists():
            raise RuntimeError(
                f"HIP extension not built: {LIBRARY_PATH} is missing "
                "(run `python -m dsa_amd.build`)"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH))
        except OSError as exc:  # pragma: no cover - depends on the host
            raise RuntimeError(f"HIP extension not built or not loadable: {exc}") from exc
        lib.dsa_last_error.restype = ctypes.c_char_p
        lib.dsa_last_error.argtypes = []
        lib.dsa_abi_version.restype = ctypes.c_int
        lib.dsa_abi_version.argtypes = []
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = argtypes
        for name, (restype, argtypes) in _RESTYPES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.dsa_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libdsa_amd ABI {version} != expected {ABI_VERSION}; rebuild")
        atexit.register(_release)
        _lib = lib
        return lib


def _release() -> None:
    """Interpreter-exit hook (registered when the library loads): waits for
    the device work still queued on this process's streams and hands the
    cached workspaces back to torch's allocator.  Python runs it before its
    own teardown and before the C exit handlers (torch's and the HIP runtime's
    destructors, the library's code-object unregistration), so that nothing
    of this package is released while they tear down."""

    try:
        if torch.cuda.is_initialized():
            with _workspace_lock:
                devices = {key[1] for key in _workspace_cache} | {torch.cuda.current_device()}
            for index in sorted(d for d in devices if d is not None):
                torch.cuda.synchronize(index)
    finally:
        with _workspace_lock:
            _workspace_cache.clear()


def call(name: str, *args) -> None:
    """Invoke a status-returning entry point; raise RuntimeError on failure."""

    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.dsa_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {status}): {message}")


def query(name: str, *args):
    """Invoke a value-returning entry point."""

    return getattr(load(), name)(*args)


def ptr(tensor: torch.Tensor | None) -> int | None:
    """Device address of a tensor (None for a missing optional argument)."""

    return None if tensor is None else tensor.data_ptr()


def stream_of(tensor: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on the tensor's device."""

    return torch.cuda.current_stream(tensor.device).cuda_stream


_workspace_cache: dict[tuple, torch.Tensor] = {}
_workspace_lock = threading.Lock()


def workspace(kind: str, device: torch.device, stream: int, need: int, *, zeroed: bool, rows: int = 0) -> torch.Tensor:
    """A device workspace of at least ``need`` bytes shared by every call of
    one ``kind`` on one stream (calls on a stream are ordered, so they never
    overlap).

    The entry points accept any workspace at least as large as they ask for,
    so one buffer serves every length.  It grows geometrically (at least
    doubling), so a decode loop whose context grows by one key per step
    reallocates O(log L) times instead of keeping a buffer per length.
    ``zeroed`` buffers are zero-filled when allocated; the entry points that
    need zeros there (a per-row region at the start of the buffer) leave them
    zeroed after every call.  That region grows with the row count, over
    space that calls with fewer rows use for other data, so zeroed buffers
    are also kept per ``rows``.
    """

    key = (kind, device.index, stream, rows if zeroed else 0)
    with _workspace_lock:
        ws = _workspace_cache.get(key)
        if ws is None or ws.numel() < need:
            size = max(int(need), 256, 2 * ws.numel() if ws is not None else 0)
            ws = (torch.zeros if zeroed else torch.empty)(size, device=device, dtype=torch.uint8)
            _workspace_cache[key] = ws
        return ws


def workspace_count() -> int:
    """Number of cached workspaces (one per kind, device and stream)."""

    return len(_workspace_cache)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None
