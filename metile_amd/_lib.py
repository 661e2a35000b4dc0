"""ctypes binding of ``libmetile_amd.so`` (the C ABI declared in ``include/metile_amd.h``).

The library is loaded from the package directory. There is no fallback: if it is missing or
fails to load, :func:`lib` raises, so no operator can silently run elsewhere.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmetile_amd.so"

MT_OK = 0
MT_ERR_INVALID_ARGUMENT = -1
MT_ERR_WORKSPACE = -2
MT_ERR_HIP = -3

MT_BF16 = 0
MT_F16 = 1

MT_QMV_STAGED = 1
MT_QMV_REGISTER = 2
MT_QMV_GEMV = 3
MT_QMV_BLOCK = 4
MT_QMV_GEMV4 = 5
MT_GEMM_STAGED = 0
MT_GEMM_RING = 1
MT_LAYOUT_MLX = 0
MT_LAYOUT_REPACKED = 1


class QmvPlan(ctypes.Structure):
    """``mt_qmv_plan``."""

    _fields_ = [("kernel", ctypes.c_int), ("ksplit", ctypes.c_int), ("strips", ctypes.c_int),
                ("tiles", ctypes.c_int), ("order", ctypes.c_int)]


class GemmPlan(ctypes.Structure):
    """``mt_gemm_plan``."""

    _fields_ = [("kernel", ctypes.c_int), ("tile_m", ctypes.c_int), ("tile_n", ctypes.c_int),
                ("ksplit", ctypes.c_int), ("order", ctypes.c_int)]


class DensePlan(ctypes.Structure):
    """``mt_dense_plan``."""

    _fields_ = [("ksplit", ctypes.c_int)]


_P = ctypes.c_void_p
_I = ctypes.c_int
_Z = ctypes.c_size_t
_QP = ctypes.POINTER(QmvPlan)
_GP = ctypes.POINTER(GemmPlan)
_DP = ctypes.POINTER(DensePlan)

# name -> (restype, argtypes); mirrors include/metile_amd.h exactly.
SIGNATURES = {
    "mt_version": (ctypes.c_char_p, []),
    "mt_last_error": (ctypes.c_char_p, []),
    "mt_affine_qmv_workspace_bytes": (_Z, [_I, _I, _I, _I, _I, _I]),
    "mt_affine_qmv": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _Z, _P]),
    "mt_affine_swiglu": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _Z,
                              _P]),
    "mt_affine_mlp_workspace_bytes": (_Z, [_I, _I, _I, _I, _I]),
    "mt_affine_mlp": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                           _I, _P, _Z, _P]),
    "mt_affine_mlp_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                                   _I, _I, _P]),
    "mt_affine_dequantize": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "mt_affine_quantize": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "mt_affine_repack": (_I, [_P, _P, _I, _I, _I, _P]),
    "mt_affine_qmv_repacked": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _Z, _P]),
    "mt_affine_swiglu_repacked": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                       _P, _Z, _P]),
    "mt_affine_mlp_repacked": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                                    _I, _I, _I, _P, _Z, _P]),
    "mt_affine_mlp_layouts": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                                   _I, _I, _I, _I, _I, _P, _Z, _P]),
    "mt_affine_gemm_workspace_bytes": (_Z, [_I, _I, _I, _I, _I]),
    "mt_affine_gemm": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _Z, _P]),
    "mt_stream_read": (_I, [_P, _Z, _P, _I, _P]),
    "mt_stream_read_blocked": (_I, [_P, _Z, _P, _I, _P]),
    "mt_dense_workspace_bytes": (_Z, [_I, _I, _I, _I]),
    "mt_dense_swiglu": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _Z, _P]),
    "mt_dense_residual_qmv": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _Z, _P]),
    "mt_affine_qmv_plan": (_I, [_I, _I, _I, _I, _I, _I, _I, _QP]),
    "mt_affine_qmv_plan_candidates": (_I, [_I, _I, _I, _I, _I, _I, _QP, _I]),
    "mt_affine_qmv_plan_set": (_I, [_I, _I, _I, _I, _I, _I, _I, _QP]),
    "mt_affine_gemm_plan": (_I, [_I, _I, _I, _I, _I, _GP]),
    "mt_affine_gemm_plan_candidates": (_I, [_I, _I, _I, _I, _GP, _I]),
    "mt_affine_gemm_plan_set": (_I, [_I, _I, _I, _I, _I, _GP]),
    "mt_dense_qmv_plan": (_I, [_I, _I, _I, _I, _DP]),
    "mt_dense_qmv_plan_candidates": (_I, [_I, _I, _I, _DP, _I]),
    "mt_dense_qmv_plan_set": (_I, [_I, _I, _I, _I, _DP]),
    "mt_plans_clear": (_I, []),
    "mt_source_digest": (ctypes.c_char_p, []),
}

_lock = threading.Lock()
_lib = None


class MetileError(RuntimeError):
    """A C-ABI call returned a failure status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m metile_amd.build` "
                    "(metile_amd has no non-HIP fallback)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def check(status: int) -> None:
    """Raise :class:`MetileError` (or ``ValueError`` for argument errors) on failure."""
    if status == MT_OK:
        return
    msg = (lib().mt_last_error() or b"").decode()
    if status == MT_ERR_INVALID_ARGUMENT:
        raise ValueError(msg)
    raise MetileError(status, msg)


def version() -> str:
    return lib().mt_version().decode()
