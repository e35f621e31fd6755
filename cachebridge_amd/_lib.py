"""ctypes binding of ``libcachebridge_hip.so`` (C ABI in ``include/cachebridge_hip.h``).

The library is built in-tree by ``cachebridge_amd.build.build_library()``.
There is no fallback: if the library is missing or cannot be loaded, every
entry point raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  -- binds torch's HIP runtime before the library loads

LIB_NAME = "libcachebridge_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

CB_OK = 0
CB_EINVAL = -22
CB_ENOMEM = -12
CB_EHIP = -5
CB_DTYPE_BF16 = 0
CB_DTYPE_F32 = 1
CB_DTYPE_F64 = 2
CB_DTYPE_F16 = 3
CB_KIND_K = 0
CB_KIND_V = 1
CB_INDEX_IDENTITY = 0
CB_INDEX_I32 = 1
CB_INDEX_I64 = 2
CB_INDEX_BLOCK_TABLE = 3
CB_MAX_WINDOW_CLASSES = 4
CB_MAX_SUPPORT = 16
CB_NOALLOC_WORKSPACE_BYTES = 16777216
CB_NOALLOC_MAX_TOKENS = 1398080

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class CbRows(ctypes.Structure):
    _fields_ = [
        ("k_layers", _c_void_p),
        ("v_layers", _c_void_p),
        ("k_base", _c_void_p),
        ("v_base", _c_void_p),
        ("layer_stride", _i64),
        ("row_stride", _i64),
        ("rows", _i64),
        ("num_layers", _i32),
        ("head_offset", _i32),
        ("heads", _i32),
        ("index_kind", _i32),
        ("index", _c_void_p),
        ("index_offset", _i64),
        ("page_size", _i32),
        ("reserved", _i32),
    ]


class CbPlanDesc(ctypes.Structure):
    _fields_ = [
        ("head_dim", _i32),
        ("support", _i32),
        ("io_dtype", _i32),
        ("num_jobs", _i32),
        ("target_layers", _i32),
        ("target_heads", _i32),
        ("job_target_layer", ctypes.POINTER(_i32)),
        ("job_target_head", ctypes.POINTER(_i32)),
        ("job_kind", ctypes.POINTER(_i32)),
        ("job_window", ctypes.POINTER(_i32)),
        ("job_source_theta", ctypes.POINTER(_i32)),
        ("job_target_theta", ctypes.POINTER(_i32)),
        ("job_source_layer", ctypes.POINTER(_i32)),
        ("job_source_head", ctypes.POINTER(_i32)),
        ("d_weight", _c_void_p),
        ("d_bias", _c_void_p),
        ("num_thetas", _i32),
        ("table_positions", _i32),
        ("d_cos", _c_void_p),
        ("d_sin", _c_void_p),
        ("num_windows", _i32),
        ("window_size", _i32 * CB_MAX_WINDOW_CLASSES),
    ]


class CbRequest(ctypes.Structure):
    _fields_ = [
        ("source", CbRows),
        ("target", CbRows),
        ("num_tokens", _i32),
        ("position_start", _i32),
        ("prefix_length", _i32),
        ("tokens_per_workgroup", _i32),
    ]


class CbSpan(ctypes.Structure):
    _fields_ = [
        ("source_offset", _i64),
        ("target_offset", _i64),
        ("num_tokens", _i32),
        ("position_start", _i32),
        ("prefix_length", _i32),
        ("reserved", _i32),
    ]


class CbPlanInfo(ctypes.Structure):
    _fields_ = [
        ("head_dim", _i32),
        ("support", _i32),
        ("io_dtype", _i32),
        ("num_jobs", _i32),
        ("target_layers", _i32),
        ("target_heads", _i32),
        ("num_groups", _i32),
        ("num_thetas", _i32),
        ("table_positions", _i32),
        ("weight_terms", _i32),
        ("device_bytes", _i64),
    ]


# Every symbol the header declares, with (restype, argtypes).
SIGNATURES = {
    "cb_last_error": (ctypes.c_char_p, []),
    "cb_abi_version": (ctypes.c_int, []),
    "cb_plan_create": (ctypes.c_int, [ctypes.POINTER(CbPlanDesc), ctypes.POINTER(_c_void_p)]),
    "cb_plan_destroy": (None, [_c_void_p]),
    "cb_plan_get_info": (ctypes.c_int, [_c_void_p, ctypes.POINTER(CbPlanInfo)]),
    "cb_plan_last_split": (ctypes.c_int, [_c_void_p, ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    "cb_map_install": (ctypes.c_int, [_c_void_p, ctypes.POINTER(CbRequest), _c_void_p]),
    "cb_batch_workspace_bytes": (ctypes.c_int, [_c_void_p, ctypes.POINTER(CbSpan), _i32,
                                                ctypes.POINTER(_i64)]),
    "cb_map_install_batch": (
        ctypes.c_int,
        [_c_void_p, ctypes.POINTER(CbRows), ctypes.POINTER(CbRows), ctypes.POINTER(CbSpan), _i32,
         _c_void_p, _i64, _c_void_p],
    ),
    "cb_map_install_batch_noalloc": (
        ctypes.c_int,
        [_c_void_p, ctypes.POINTER(CbRows), ctypes.POINTER(CbRows), ctypes.POINTER(CbSpan), _i32,
         _c_void_p],
    ),
    "cb_copy_rows": (
        ctypes.c_int,
        [ctypes.POINTER(CbRows), ctypes.POINTER(CbRows), _i32, _i32, _i32, _i32, _c_void_p, _c_void_p],
    ),
    "cb_plan_read_errors": (ctypes.c_int, [_c_void_p, ctypes.POINTER(_i32), _c_void_p]),
    "cb_delta_state_transform": (
        ctypes.c_int,
        [_i32, _i64, _i32, _i32, _i32, _i32, _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64,
         _c_void_p, _i64, _c_void_p],
    ),
}

_LIB: ctypes.CDLL | None = None


class CacheBridgeHipError(RuntimeError):
    """A C-ABI call returned a HIP runtime failure."""


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is not built.

    ``CACHEBRIDGE_HIP_LIBRARY`` names an alternative build of the same ABI.
    """
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    override = os.environ.get("CACHEBRIDGE_HIP_LIBRARY")
    lib_path = Path(path) if path is not None else Path(override) if override else LIB_PATH
    if not lib_path.exists():
        raise RuntimeError(
            f"{lib_path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "or `python -m cachebridge_amd.build` first (there is no CPU fallback)"
        )
    lib = ctypes.CDLL(str(lib_path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.cb_abi_version() != 1:
        raise RuntimeError("libcachebridge_hip ABI version mismatch")
    if path is None:
        _LIB = lib
    return lib


def check(rc: int) -> None:
    """Raise the Python error matching a C-ABI return code."""
    if rc == CB_OK:
        return
    message = load().cb_last_error().decode(errors="replace")
    if rc == CB_EINVAL:
        raise ValueError(message)
    if rc == CB_ENOMEM:
        raise MemoryError(message)
    raise CacheBridgeHipError(message)


def stream_handle(stream: torch.cuda.Stream | None = None) -> int:
    """Raw HIP stream handle of ``stream`` (default: torch's current stream)."""
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)
