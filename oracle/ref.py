"""ctypes access to oracle/_ref/libref_w4a8.so -- TEST INFRASTRUCTURE ONLY.

The library is the reference's own C++ CPU reference
(int4_cube_lab/host/gemm_ref.cpp, bf16.h, npu_ops/kernel/mg_kgeom.h) compiled by
oracle/Makefile.  ``available()`` is False when it was not built (the
reference checkout is absent); tests that need it skip.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import numpy as np

REF_DIR = Path(__file__).resolve().parent / "_ref"
LIB = REF_DIR / "libref_w4a8.so"
RAGGED_TEST = REF_DIR / "ragged_layout_test"

_lib: Optional[ctypes.CDLL] = None
_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_U32 = ctypes.c_uint32


def available() -> bool:
    return LIB.exists()


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        h = ctypes.CDLL(str(LIB))
        h.ref_fp32_to_bf16.argtypes = [_P, _P, _SZ]
        for name in ("ref_num_groups", "ref_kpad"):
            getattr(h, name).argtypes = [_U32, _U32]
            getattr(h, name).restype = _U32
        h.ref_group_real.argtypes = [_U32, _U32, _U32]
        h.ref_group_real.restype = _U32
        h.ref_group_offset.argtypes = [_U32, _U32]
        h.ref_group_offset.restype = _U32
        h.ref_pack_int4.argtypes = [_P, _SZ, _SZ, _P]
        h.ref_pack_int4_grouped.argtypes = [_P, _SZ, _U32, _U32, _P]
        h.ref_weight_ksum_per_group.argtypes = [_P, _SZ, _SZ, _SZ, _P]
        h.ref_act_ksum_neg_per_group.argtypes = [_P, _SZ, _SZ, _SZ, _P]
        h.ref_split_planes_grouped.argtypes = [_P, _SZ, _U32, _U32, _P, _P]
        h.ref_midgroup_gemm.argtypes = [_P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32]
        h.ref_perchannel_gemm.argtypes = [_P, _P, _P, _P, _P, _U32, _U32, _U32]
        h.ref_set_threads.argtypes = [ctypes.c_int]
        h.ref_max_threads.restype = ctypes.c_int
        _lib = h
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def fp32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().ref_fp32_to_bf16(_ptr(x), _ptr(out), x.size)
    return out


def pack_int4_grouped(codes: np.ndarray, group: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.int8)
    rows, K = codes.shape
    out = np.empty((rows, lib().ref_kpad(K, group) // 2), np.int8)
    lib().ref_pack_int4_grouped(_ptr(codes), rows, K, group, _ptr(out))
    return out


def split_planes_grouped(a_q: np.ndarray, group: int):
    """SplitInt8ToInt4PlanesGrouped (gemm_ref.cpp:62-90): packed (hi, lo) int4
    planes [rows, kpad/2] with a = 16*hi + lo + 8 in the padded K layout."""
    a_q = np.ascontiguousarray(a_q, np.int8)
    rows, K = a_q.shape
    kp = lib().ref_kpad(K, group)
    hi = np.empty((rows, kp // 2), np.int8)
    lo = np.empty((rows, kp // 2), np.int8)
    lib().ref_split_planes_grouped(_ptr(a_q), rows, K, group, _ptr(hi), _ptr(lo))
    return hi, lo


def act_ksum_neg(a_q: np.ndarray, group: int) -> np.ndarray:
    """ActKSumNegPerGroup (gemm_ref.cpp): -sum_{k in g} A per (group, row), int32 [G, M]."""
    a_q = np.ascontiguousarray(a_q, np.int8)
    rows, K = a_q.shape
    G = lib().ref_num_groups(K, group)
    out = np.empty((G, rows), np.int32)
    lib().ref_act_ksum_neg_per_group(_ptr(a_q), rows, K, group, _ptr(out))
    return out


def weight_ksum(w: np.ndarray, group: int) -> np.ndarray:
    """WeightKSumPerGroup (gemm_ref.cpp): sum_{k in g} W per (group, column), int32 [G, N]."""
    w = np.ascontiguousarray(w, np.int8)
    rows, K = w.shape
    G = lib().ref_num_groups(K, group)
    out = np.empty((G, rows), np.int32)
    lib().ref_weight_ksum_per_group(_ptr(w), rows, K, group, _ptr(out))
    return out


def midgroup_gemm(a_q: np.ndarray, a_scale_g: np.ndarray, w_codes: np.ndarray, w_scale_g: np.ndarray,
                  group: int, w_zero_g: Optional[np.ndarray] = None) -> np.ndarray:
    """ReferenceMidGroupGemm (gemm_ref.cpp:199-240): bf16 bits [M, N].

    a_scale_g [G, M], w_scale_g / w_zero_g [G, N] as bf16 bits.
    """
    a_q = np.ascontiguousarray(a_q, np.int8)
    w_codes = np.ascontiguousarray(w_codes, np.int8)
    a_scale_g = np.ascontiguousarray(a_scale_g, np.uint16)
    w_scale_g = np.ascontiguousarray(w_scale_g, np.uint16)
    M, K = a_q.shape
    N = w_codes.shape[0]
    y = np.empty((M, N), np.uint16)
    wz = None if w_zero_g is None else np.ascontiguousarray(w_zero_g, np.uint16)
    lib().ref_midgroup_gemm(_ptr(a_q), _ptr(a_scale_g), _ptr(w_codes), _ptr(w_scale_g),
                            None if wz is None else _ptr(wz), _ptr(y), M, N, K, group, M)
    return y


def set_threads(n: int) -> int:
    """Set the OpenMP team size of the reference's loops; returns the size now in effect."""
    lib().ref_set_threads(int(n))
    return int(lib().ref_max_threads())


def perchannel_gemm(a_q: np.ndarray, a_scale: np.ndarray, w_codes: np.ndarray, w_scale: np.ndarray) -> np.ndarray:
    """ReferencePerchannelGemm (gemm_ref.cpp:154-179): bf16 bits [M, N] of
    bf16(float(sum_k a*w) * as[m] * ws[n]); a_scale [M], w_scale [N] bf16 bits."""
    a_q = np.ascontiguousarray(a_q, np.int8)
    w_codes = np.ascontiguousarray(w_codes, np.int8)
    a_scale = np.ascontiguousarray(a_scale, np.uint16)
    w_scale = np.ascontiguousarray(w_scale, np.uint16)
    M, K = a_q.shape
    N = w_codes.shape[0]
    y = np.empty((M, N), np.uint16)
    lib().ref_perchannel_gemm(_ptr(a_q), _ptr(a_scale), _ptr(w_codes), _ptr(w_scale), _ptr(y), M, N, K)
    return y


def num_groups(K: int, group: int) -> int:
    return int(lib().ref_num_groups(K, group))


def kpad(K: int, group: int) -> int:
    return int(lib().ref_kpad(K, group))


def group_offset(g: int, group: int) -> int:
    return int(lib().ref_group_offset(g, group))


def group_real(g: int, K: int, group: int) -> int:
    return int(lib().ref_group_real(g, K, group))
