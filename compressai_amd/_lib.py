"""ctypes binding of libvq2_amd.so (the C ABI declared in include/vq2_amd.h).

The library is built in-tree (``python -m compressai_amd.build`` or
``__graft_entry__.build()``) and loaded from this package directory.  There is
no fallback: if the library is missing, every entry raises.
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libvq2_amd.so"
HEADER_PATH = PKG_DIR.parent / "include" / "vq2_amd.h"

DT_F32, DT_F16, DT_BF16 = 0, 1, 2
S2_NONE, S2_U8, S2_U16 = 0, 1, 2
ID_I32, ID_I64 = 0, 1
OK, ERR_ARG, ERR_HIP, ERR_UNSUPPORTED = 0, 1, 2, 3
NOALLOC_SCRATCH_BYTES = 16 << 20  # VQ2_NOALLOC_SCRATCH_BYTES

_vp, _i64, _i32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float

# argument types of every exported entry, in header order
SIGNATURES = {
    "vq2_version": ([], _i32),
    "vq2_last_error": ([], ctypes.c_char_p),
    "vq2_gemv": ([_vp, _i32, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64,
                  _i64, _i64, _f32, _vp], _i32),
    "vq2_gemv_rht": ([_vp, _i32, _i64, _i64, _vp, _vp, _i64, _f32, _i32, _vp, _i32, _vp, _vp, _i32, _i32, _i32,
                      _i64, _f32, _vp], _i32),
    "vq2_moe_gate_up_rht": ([_vp, _i32, _i64, _vp, _vp, _i64, _f32, _vp, _i32, _i64, _vp, _i64, _vp, _i32, _vp,
                             _i32, _vp, _i32, _i64, _i64, _i64, _f32, _vp], _i32),
    "vq2_moe_router_gate_up_rht": ([_vp, _i32, _i64, _vp, _vp, _i64, _f32, _vp, _i32, _i64, _i32, _vp, _i32, _i64,
                                    _vp, _i64, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _f32, _vp, _vp,
                                    _vp], _i32),
    "vq2_moe_down_swiglu_combine": ([_vp, _i32, _i64, _vp, _vp, _i64, _f32, _vp, _i32, _vp, _i64, _i64, _vp, _i64,
                                     _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _f32, _vp], _i32),
    "vq2_moe_gate_up_rht_16_8": ([_vp, _i32, _i64, _vp, _vp, _i64, _f32, _vp, _i32, _i64, _vp, _vp, _i64, _vp,
                                  _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _f32, _vp], _i32),
    "vq2_moe_down_swiglu_combine_16_8": ([_vp, _i32, _i64, _vp, _vp, _i64, _f32, _vp, _i32, _vp, _i64, _i64, _vp,
                                          _vp, _i64, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _f32,
                                          _i32, _vp], _i32),
    "vq2_gemm_small_m_workspace": ([_i64, _i64, _i64], ctypes.c_size_t),
    "vq2_gemm_small_m_argmax_workspace": ([_i64, _i64, _i64], ctypes.c_size_t),
    "vq2_gemm_small_m_argmax": ([_vp, _i32, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _f32,
                                 _vp, ctypes.c_size_t, _vp, _vp, _vp], _i32),
    "vq2_gemm_small_m": ([_vp, _i32, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64,
                          _i64, _i64, _f32, _vp, ctypes.c_size_t, _vp], _i32),
    "vq2_gemm_small_m_noalloc": ([_vp, _i32, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64,
                                  _i64, _i64, _f32, _vp], _i32),
    "vq2_moe_grouped": ([_vp, _i32, _i64, _i64, _vp, _i32, _i64, _vp, _i64, _vp, _i32, _vp, _i32, _vp, _i32,
                         _i64, _i64, _i64, _f32, _vp], _i32),
    "vq2_moe_down_combine": ([_vp, _i32, _vp, _i32, _vp, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _i32,
                              _vp, _i32, _i64, _i64, _i64, _f32, _vp], _i32),
    "vq2_rht": ([_vp, _i32, _i64, _vp, _i32, _i64, _vp, _vp, _i64, _i64, _i64, _f32, _i32, _vp], _i32),
    "vq2_swiglu_rht": ([_vp, _i32, _i64, _i64, _vp, _i32, _i64, _vp, _vp, _i64, _i64, _f32, _vp], _i32),
    "vq2_router_topk": ([_vp, _i32, _i64, _i64, _i32, _vp, _i32, _i64, _vp, _i32, _i64, _vp, _vp, _vp],
                        _i32),
    "vq2_argmax_rows": ([_vp, _i32, _i64, _i64, _vp, _vp, _vp], _i32),
    "vq2_gemv_argmax": ([_vp, _i32, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _vp, _i32, _i64, _i64,
                         _f32, _vp, _vp, _vp, _vp], _i32),
    "vq2_sorted_rows_per_chunk": ([_i64, _i64, _i64], _i64),
    "vq2_sorted_pack": ([_vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i32], _i32),
    "vq2_sorted_gemv_workspace": ([_vp, _i32, _i32], ctypes.c_size_t),
    "vq2_sorted_gemv": ([_vp, _i32, _vp, _vp, _i64, _f32, _i32, _vp, _vp, _vp, _i32, _i32, _i32, _i64, _f32, _i32,
                         _vp, ctypes.c_size_t, _vp], _i32),
    "vq2_sorted_gemv_argmax_workspace": ([_vp], ctypes.c_size_t),
    "vq2_sorted_gemv_argmax": ([_vp, _i32, _vp, _vp, _i64, _f32, _vp, _vp, _vp, _i32, _i32, _i64, _f32, _vp,
                                ctypes.c_size_t, _vp, _vp, _vp], _i32),
    "vq2_sorted_gemm_batch_workspace": ([_vp, _i32, _i64, _i32], ctypes.c_size_t),
    "vq2_sorted_gemm_batch": ([_vp, _i32, _i64, _i64, _i32, _vp, _vp, _vp, _i32, _i32, _i32, _i64, _f32, _i32, _vp,
                               ctypes.c_size_t, _vp], _i32),
    "vq2_sorted_gemm_batch_argmax_workspace": ([_vp, _i64], ctypes.c_size_t),
    "vq2_sorted_gemm_batch_argmax": ([_vp, _i32, _i64, _i64, _vp, _vp, _vp, _i32, _i32, _i64, _f32, _vp,
                                      ctypes.c_size_t, _vp, _vp, _vp], _i32),
    "vq2_sorted_pack_pool": ([_vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i32], _i32),
    "vq2_sorted_moe_workspace": ([_i64, _i32, _i64, _i64, _i32, _i32], ctypes.c_size_t),
    "vq2_sorted_moe": ([_vp, _i32, _i64, _i32, _vp, _i32, _vp, _vp, _i32, _i64, _i32, _i64, _vp, _i32, _vp, _vp,
                        _i64, _i64, _i64, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _i32, _i32, _i32, _vp,
                        ctypes.c_size_t, _vp], _i32),
    "vq2_sorted_moe_status": ([_vp, _i32, _vp], _i32),
    "vq2_sorted_moe_set_wait": ([_i64, _i32], _i32),
    "vq2_pager_lds_bytes": ([_i64, _i64, _i64], ctypes.c_size_t),
    "vq2_pager_step": ([_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "vq2_pager_copy": ([_vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _i32, _vp], _i32),
    "vq2_dequant_rows": ([_vp, _vp, _i32, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _vp, _vp], _i32),
    "vq2_decode_idx": ([_vp, _i32, _i64, _vp, _vp], _i32),
    "vq2_unpack_fixed": ([_vp, _i64, _i32, _i64, _vp, _vp], _i32),
}

_lib = None


class Vq2Error(RuntimeError):
    """A libvq2_amd entry returned a non-zero status."""


class Seg(ctypes.Structure):
    """struct vq2_seg of include/vq2_amd.h"""
    _fields_ = [("idx0", ctypes.c_void_p), ("idx1", ctypes.c_void_p), ("scale", ctypes.c_void_p),
                ("y", ctypes.c_void_p), ("out_rows", ctypes.c_int64), ("y_stride", ctypes.c_int64)]


class SortedMat(ctypes.Structure):
    """struct vq2_sorted_mat of include/vq2_amd.h"""
    _fields_ = [("entries", ctypes.c_void_p), ("iters_per_chunk", ctypes.c_int64), ("stage1_iters", ctypes.c_int64),
                ("n_iters", ctypes.c_int64), ("rows_per_chunk", ctypes.c_int64), ("has_stage2", ctypes.c_int),
                ("scale", ctypes.c_void_p),
                ("y", ctypes.c_void_p), ("out_rows", ctypes.c_int64)]


class SortedPool(ctypes.Structure):
    """struct vq2_sorted_pool of include/vq2_amd.h"""
    _fields_ = [("entries", ctypes.c_void_p), ("iters_per_chunk", ctypes.c_int64), ("n_iters", ctypes.c_int64),
                ("rows_per_chunk", ctypes.c_int64), ("rows", ctypes.c_int64), ("ng", ctypes.c_int64),
                ("scale", ctypes.c_void_p), ("scale_dt", ctypes.c_int), ("stage1_iters", ctypes.c_int64),
                ("has_stage2", ctypes.c_int), ("cb1", ctypes.c_void_p)]


class RotTables(ctypes.Structure):
    """struct vq2_rot_tables of include/vq2_amd.h"""
    _fields_ = [("perm", ctypes.c_void_p), ("sign", ctypes.c_void_p), ("hb", ctypes.c_int64),
                ("scale", ctypes.c_float)]


def header_symbols() -> list[str]:
    """Names of the functions declared in include/vq2_amd.h."""
    text = HEADER_PATH.read_text()
    return re.findall(r"^\s*(?:int|int64_t|size_t|const char\*)\s+(vq2_\w+)\s*\(", text, flags=re.M)


def load():
    """Load the library (once).  Raises ImportError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} not found: build the HIP extension first "
            "(python -c 'import __graft_entry__ as g; g.build()')")
    L = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_LOCAL if hasattr(os, "RTLD_LOCAL") else 0)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return _lib


def check(status: int, what: str = "") -> None:
    if status != OK:
        msg = load().vq2_last_error().decode(errors="replace")
        raise Vq2Error(f"{what or 'libvq2_amd'} failed (status {status}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)
