"""ctypes binding of the C ABI in include/w4a8_amd.h.

The library path is ``_lib/libw4a8_amd.so`` inside this package, or the file
named by the ``W4A8_AMD_LIB`` environment variable (the reference selects its
op library the same way through ``W4A8_OPS_LIB``,
npu_ops/python/w4a8_ops.py:39-58).  A missing library raises: there is no
fallback implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "_lib" / "libw4a8_amd.so"
ABI_VERSION = 10

W4A8_DT_F16 = 0
W4A8_DT_BF16 = 1
NOALLOC_SCRATCH_BYTES = 8 << 20   # W4A8_NOALLOC_SCRATCH_BYTES

# Every symbol include/w4a8_amd.h declares, with its ctypes signature.
_VP, _I64, _I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
SIGNATURES = {
    "w4a8_abi_version": (_I, []),
    "w4a8_last_error": (ctypes.c_char_p, []),
    "w4a8_stream_capture_id": (_I, [_VP, ctypes.POINTER(ctypes.c_ulonglong)]),
    "w4a8_read_floor": (_I, [_VP, _I64, _VP, _VP]),
    "w4a8_quant_act": (_I, [_VP, _I64, _VP, _I64, _VP, _I64, _I64, _I64, _VP]),
    "w4a8_repacked_weight_bytes": (_I64, [_I64, _I64, _I64]),
    "w4a8_repacked_scale_bytes": (_I64, [_I64, _I64, _I64]),
    "w4a8_repack": (_I, [_VP, _VP, _I, _VP, _VP, _I64, _I64, _I64, _VP]),
    "w4a8_gemm_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "w4a8_gemm_row_chunk": (_I64, [_I64, _I64]),
    "w4a8_gemm": (_I, [_VP, _I64, _VP, _VP, _VP, _I, _VP, _I64, _I64, _I64, _I64, _I64, _VP, _I64, _VP]),
    "w4a8_gemm_noalloc": (_I, [_VP, _I64, _VP, _VP, _VP, _I, _VP, _I64, _I64, _I64, _I64, _I64, _VP]),
    "w4a8_gemm_swiglu": (_I, [_VP, _I64, _VP, _VP, _VP, _I, _VP, _I64, _I64, _I64, _I64, _I64, _VP, _I64, _VP]),
    "w4a8_linear_fused": (_I, [_VP, _I64, _I64, _I64, _I64, _I64]),
    "w4a8_linear": (_I, [_VP, _I64, _VP, _VP, _I, _VP, _I64, _VP, _I64, _VP, _I64, _I64, _I64, _I64, _VP, _I64, _VP]),
    "w4a8_midgroup_quant_a": (_I, [_VP, _I64, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _VP]),
    "w4a8_midgroup_gemm": (_I, [_VP, _VP, _VP, _VP, _I64, _I64, _VP, _VP, _VP, _VP, _I64, _VP, _I64, _I64, _I64,
                                _VP]),
    "w4a8_midgroup_gemm_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "w4a8_midgroup_tiles_bytes": (_I64, [_I64, _I64, _I64]),
    "w4a8_midgroup_tile_weights": (_I, [_VP, _VP, _I64, _I64, _I64, _VP]),
    "w4a8_midgroup_gemm_tiled": (_I, [_VP, _VP, _VP, _VP, _I64, _I64, _VP, _VP, _VP, _VP, _I64, _VP, _I64, _I64, _I64,
                                      _VP, _I64, _VP]),
    "w4a8_midgroup_gemm_ws": (_I, [_VP, _VP, _VP, _VP, _I64, _I64, _VP, _VP, _VP, _VP, _I64, _VP, _I64, _I64, _I64,
                                   _VP, _I64, _VP]),
    "w4a8_rmsnorm_quant": (_I, [_VP, _I64, _VP, _I64, _VP, ctypes.c_float, _VP, _I64, _VP, _I64, _VP, _I64, _VP,
                                _I64, _I64, _I64, _VP]),
    "w4a8_gemm_debug_partials": (_I, [_VP, _I64, _VP, _VP, _VP, _I, _VP, _I64, _VP, _I64, _I64, _I64, _I64,
                                      _VP, _I64, _VP]),
    "w4a8_rope_kv": (_I, [_VP, _I64, _VP, _VP, _VP, _I64, _I64, _VP, _VP, _VP, ctypes.POINTER(_I64), _VP,
                          ctypes.POINTER(_I64), _I64, _I64, _I64, _I64, _I64, _VP]),
    "w4a8_attention": (_I, [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                            ctypes.c_float, _VP, _I64, _VP]),
    "w4a8_attention_rope": (_I, [_VP, _I64, _VP, _VP, _VP, _I64, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64,
                                 _I64, _I64, ctypes.c_float, _VP, _I64, _VP]),
    "w4a8_attention_chunks_per_split": (_I64, [_I64, _I64, _I64, _I64]),
    "w4a8_attention_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64, _I64]),
}

STATUS_NAMES = {0: "OK", 1: "NULL", 2: "SHAPE", 3: "DTYPE", 4: "ALIGN", 5: "UNSUPPORTED", 6: "WORKSPACE",
                7: "HIP"}

_lock = threading.Lock()
_lib = None


def lib_path() -> Path:
    override = os.environ.get("W4A8_AMD_LIB")
    return Path(override) if override else LIB_PATH


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not path.exists():
                raise FileNotFoundError(
                    f"W4A8 HIP library not found at {path}; build it with "
                    f"`python -c 'import __graft_entry__ as g; g.build()'` or point W4A8_AMD_LIB at it")
            handle = ctypes.CDLL(str(path))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            ver = handle.w4a8_abi_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"{path} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Raise RuntimeError for a non-zero status, with the library's message."""
    if status != 0:
        msg = lib().w4a8_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{what} failed ({STATUS_NAMES.get(status, status)}): {msg}")
