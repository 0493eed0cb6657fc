"""ctypes binding of libung_hip.so (the C ABI declared in include/ung_hip.h).

Loading fails loudly when the library has not been built: there is no CPU or
PyTorch fallback for any entry point of the path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libung_hip.so")

UNG_HIP_OK = 0
UNG_HIP_EINVAL = -1
UNG_HIP_EDEVICE = -2
UNG_HIP_ESTATE = -3


class UngHipError(RuntimeError):
    """Raised for a non-zero return of a C ABI entry point (carries the code)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class Stats(C.Structure):
    _fields_ = [
        ("wall_ms", C.c_double),
        ("plan_ms", C.c_double),
        ("h2d_ms", C.c_double),
        ("kernel_ms", C.c_double),
        ("select_ms", C.c_double),
        ("merge_ms", C.c_double),
        ("fallback_ms", C.c_double),
        ("d2h_ms", C.c_double),
        ("pairs", C.c_uint64),
        ("rows", C.c_uint64),
        ("work_items", C.c_uint64),
        ("select_launches", C.c_uint64),
        ("fallback_rows", C.c_uint64),
        ("padded_pairs", C.c_uint64),
        ("select_bytes", C.c_uint64),
        ("allocations", C.c_uint64),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


_vp = C.c_void_p
_u32 = C.c_uint32
_u64 = C.c_uint64
_i32 = C.c_int32
_dbl = C.c_double
_int = C.c_int

# name -> (restype, argtypes); every symbol declared in include/ung_hip.h
SIGNATURES = {
    "ung_hip_last_error": (C.c_char_p, []),
    "ung_hip_version": (C.c_char_p, []),
    "ung_hip_create": (_int, [_int, C.POINTER(_vp)]),
    "ung_hip_destroy": (_int, [_vp]),
    "ung_hip_prepare_vectors": (_int, [_vp, _vp, _u64, _u32, _vp]),
    "ung_hip_prepare_vectors_device": (_int, [_vp, _vp, _u64, _u32, _vp]),
    "ung_hip_release_vectors": (_int, [_vp]),
    "ung_hip_cross_topk": (_int, [_vp, _u32, _vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp]),
    "ung_hip_cross_topk_device": (_int, [_vp, _u32, _vp, _vp, _vp, _u32, _vp]),
    "ung_hip_cross_result_device": (_int, [_vp, _vp, _vp]),
    "ung_hip_cross_topk_noalloc": (_int, [_vp, _u32, _vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp]),
    "ung_hip_download_cross": (_int, [_vp, _vp, _vp, _vp, _vp]),
    "ung_hip_additional_edges": (_int, [_vp, _u32, _vp, _vp, _vp, _u32, _vp, _vp, _vp, _u64, C.POINTER(_u64), _vp]),
    "ung_hip_group_knn": (_int, [_vp, _u32, _vp, _vp, _u32, _vp, _vp, _vp]),
    "ung_hip_group_knn_device": (_int, [_vp, _u32, _vp, _vp, _u32, _vp]),
    "ung_hip_group_result_device": (_int, [_vp, _vp, _vp, _vp]),
    "ung_hip_download_group": (_int, [_vp, _vp, _vp, _vp]),
    "ung_hip_result_shape": (_int, [_vp, _int, C.POINTER(_u64), C.POINTER(_u32), C.POINTER(_u32)]),
    "ung_hip_rescanned_rows": (_int, [_vp, _int, _vp, _u64, C.POINTER(_u64)]),
    "ung_hip_pack_anchor_rows": (_int, [_vp, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _vp, _vp]),
    "ung_hip_prune_group_graph": (_int, [_vp, _u32, _u32, _u32, C.c_float, _vp, _vp, _vp]),
    "ung_hip_cross_intra_begin": (_int, [_vp, _u32, _vp, _vp, _vp, _u32, _u32, _vp, _vp, _u32, _vp]),
    "ung_hip_intra_end": (_int, [_vp, _vp]),
    "ung_hip_synchronize": (_int, [_vp]),
    "ung_hip_selftest_mfma": (_int, [_vp, C.POINTER(_dbl)]),
    "ung_hip_debug_partial_rows": (_int, [_vp, _u64, _vp, _vp, _vp, C.POINTER(_u64), C.POINTER(_dbl),
                                          C.POINTER(_dbl)]),
    "ung_hip_debug_partial_bounds": (_int, [_vp, _u64, _vp, _vp, _vp, _vp, C.POINTER(_u64)]),
    "ung_divide_groups": (_int, [_u64, _vp, _vp, _vp, _vp, _vp, C.POINTER(_u32)]),
    "ung_group_label_sets": (_int, [_u64, _vp, _vp, _vp, _vp, _u32, _vp, _vp, _u64]),
    "ung_lng_build": (_int, [_u32, _vp, _vp, _vp, _vp, _u64, C.POINTER(_u64), _int]),
    "ung_reorder_rows": (_int, [_vp, _u64, _u32, _vp, _vp, _int]),
    "ung_assemble_graph_csr": (_int, [_u64, _u32, _vp, _vp, _vp, _int, _vp, _u32, _u32, _vp, _vp, _vp, _vp, _vp,
                                      _u64, C.POINTER(_u64), _int]),
    "ung_graph_save_text": (_int, [C.c_char_p, _u64, _vp, _vp, _int]),
    "ung_count_pairs": (_int, [_u32, _vp, _vp, _vp, _u32, _u32, C.POINTER(_u64), C.POINTER(_u64)]),
    "ung_synth_vectors": (_int, [_u64, _u32, _u32, C.c_float, C.c_float, _int, _u64, _u64, _vp, _int]),
    "ung_synth_labels": (_int, [_u64, _int, _u32, _u32, _u32, _dbl, _u64, _vp, _vp, _int]),
}

_LIB = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libung_hip.so once; raises if it is missing (no fallback path)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(the UNG HIP path has no CPU fallback)")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def last_error() -> str:
    return load().ung_hip_last_error().decode(errors="replace")


def check(rc: int) -> None:
    if rc != UNG_HIP_OK:
        raise UngHipError(rc, last_error())


def ptr(a) -> int | None:
    """Address of a numpy array's data (None for None)."""
    if a is None:
        return None
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return a.ctypes.data


def u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint32)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)
