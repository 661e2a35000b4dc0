"""Dense 16-bit small-batch projections on torch tensors (gfx950 HIP kernels via the C ABI).

Mirrors meTile's dense MLX backends (``metile/backends/mlx_dense.py``,
``mlx_dense_swiglu.py``, ``mlx_dense_residual.py``): ``DenseWeight`` stands in for
``MLXDenseWeight`` and ``mlx_dense_swiglu`` / ``mlx_dense_residual_qmv`` keep the reference
names, arguments and ``ValueError``/``TypeError`` guards. Every output row is bit-identical to
running that row alone (the reduction order of each output depends only on the plan of its
(K, N), which serves every row count). With ``autotune`` the entries first resolve that plan
(``metile_amd.tuning.ensure_dense_plan``: measured once per shape over several row counts,
persisted), as the reference's tuned dense entries do.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .quantized import _require_device, _stream_handle, workspace

_DTYPES = {torch.bfloat16: _lib.MT_BF16, torch.float16: _lib.MT_F16}


@dataclass(frozen=True)
class DenseWeight:
    """A dense output-major ``[N, K]`` weight and its logical ``shape = (K, N)``.

    Counterpart of ``MLXDenseWeight`` (``metile/backends/mlx_dense.py:56-74``). The gfx950
    kernels read the native output-major layout directly, so no K-major copy is kept.
    """

    native_weight: torch.Tensor
    shape: tuple[int, int]

    @classmethod
    def from_torch(cls, weight: torch.Tensor) -> "DenseWeight":
        if weight.ndim != 2:
            raise ValueError("dense weights must have shape [output, input]")
        if weight.dtype not in (torch.bfloat16, torch.float16):
            raise TypeError("dense weights must use bfloat16 or float16")
        return cls(weight.contiguous(), (weight.shape[1], weight.shape[0]))


def dense_swiglu(values, gate_weight, up_weight):
    """Typed SwiGLU of two dense projections; ``gate_weight``/``up_weight`` are ``[N, K]``."""
    _require_device(values, gate_weight, up_weight)
    if values.dtype not in _DTYPES:
        raise TypeError("dense SwiGLU requires bfloat16 or float16")
    if gate_weight.dtype != values.dtype or up_weight.dtype != values.dtype:
        raise TypeError("dense SwiGLU requires matching activation and weight dtypes")
    if gate_weight.shape != up_weight.shape or gate_weight.shape[1] != values.shape[-1]:
        raise ValueError("expected values[..., K] and matching [N, K] gate/up weights")
    k = values.shape[-1]
    n = gate_weight.shape[0]
    lead = tuple(values.shape[:-1])
    x = values.reshape(-1, k).contiguous()
    m = x.shape[0]
    out = torch.empty(*lead, n, dtype=values.dtype, device=values.device)
    if m == 0:
        return out
    g, u = gate_weight.contiguous(), up_weight.contiguous()
    lib = _lib.lib()
    need = lib.mt_dense_workspace_bytes(m, k, n, 2)
    ws = workspace(values.device, need) if need else None
    _lib.check(lib.mt_dense_swiglu(
        x.data_ptr(), g.data_ptr(), u.data_ptr(), out.data_ptr(), m, k, n, _DTYPES[values.dtype],
        None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
        _stream_handle(values.device)))
    return out


def dense_qmv(values, weight, residual=None):
    """``T(T(values @ weight.T) + residual)``, or ``T(values @ weight.T)`` without a residual."""
    _require_device(values, weight, residual)
    if values.dtype not in _DTYPES:
        raise TypeError("dense residual QMV requires bfloat16 or float16")
    if weight.dtype != values.dtype or (residual is not None and residual.dtype != values.dtype):
        raise TypeError("dense residual QMV requires matching input dtypes")
    if weight.ndim != 2 or weight.shape[1] != values.shape[-1]:
        raise ValueError("dense residual QMV input features must match the weight")
    k = values.shape[-1]
    n = weight.shape[0]
    lead = tuple(values.shape[:-1])
    if residual is not None and tuple(residual.shape) != (*lead, n):
        raise ValueError("dense residual QMV residual shape must match the projected output")
    x = values.reshape(-1, k).contiguous()
    m = x.shape[0]
    out = torch.empty(*lead, n, dtype=values.dtype, device=values.device)
    if m == 0:
        return out
    w = weight.contiguous()
    res = None if residual is None else residual.reshape(m, n).contiguous()
    lib = _lib.lib()
    need = lib.mt_dense_workspace_bytes(m, k, n, 1)
    ws = workspace(values.device, need) if need else None
    _lib.check(lib.mt_dense_residual_qmv(
        x.data_ptr(), w.data_ptr(), None if res is None else res.data_ptr(), out.data_ptr(), m,
        k, n, _DTYPES[values.dtype], None if ws is None else ws.data_ptr(),
        0 if ws is None else ws.numel(), _stream_handle(values.device)))
    return out


def mlx_dense_swiglu(values, gate_weight, up_weight, *, paired_weight=None, autotune=True):
    """Drop-in for ``mlx_dense_swiglu`` with the reference's guards
    (``metile/backends/mlx_dense_swiglu.py:424-447``). ``paired_weight`` (an interleaved
    ``[N, K, 2]`` copy used by one of the reference's Metal schedules) is validated and not
    needed: the gfx950 kernel streams gate and up from their own matrices."""
    if not isinstance(gate_weight, DenseWeight) or not isinstance(up_weight, DenseWeight):
        raise TypeError("gate_weight and up_weight must be DenseWeight values")
    if gate_weight.shape != up_weight.shape:
        raise ValueError("dense SwiGLU gate and up weights must have matching shapes")
    if values.ndim < 2 or values.shape[-1] != gate_weight.shape[0]:
        raise ValueError("expected values[..., K] and matching KxN gate/up weights")
    if (values.dtype != gate_weight.native_weight.dtype
            or values.dtype != up_weight.native_weight.dtype):
        raise TypeError("dense SwiGLU requires matching activation and weight dtypes")
    if values.dtype not in _DTYPES:
        raise TypeError("dense SwiGLU requires bfloat16 or float16")
    if paired_weight is not None and (
            tuple(paired_weight.shape) != (gate_weight.shape[1], gate_weight.shape[0], 2)
            or paired_weight.dtype != values.dtype):
        raise ValueError("paired dense SwiGLU weight must have shape [N, K, 2] and matching dtype")
    if autotune:
        from . import tuning

        tuning.ensure_dense_plan([gate_weight.native_weight, up_weight.native_weight],
                                 values.dtype)
    return dense_swiglu(values, gate_weight.native_weight, up_weight.native_weight)


def mlx_dense_residual_qmv(values, weight, residual, *, autotune=True):
    """Drop-in for ``mlx_dense_residual_qmv`` with the reference's guards
    (``metile/backends/mlx_dense_residual.py:276-288``)."""
    if values.ndim < 2 or weight.ndim != 2 or residual.ndim != values.ndim:
        raise ValueError("dense residual QMV requires rank-compatible values, weight, and residual")
    if values.shape[-1] != weight.shape[1]:
        raise ValueError("dense residual QMV input features must match the weight")
    if tuple(residual.shape) != (*values.shape[:-1], weight.shape[0]):
        raise ValueError("dense residual QMV residual shape must match the projected output")
    if values.dtype != weight.dtype or values.dtype != residual.dtype:
        raise TypeError("dense residual QMV requires matching input dtypes")
    if values.dtype not in _DTYPES:
        raise TypeError("dense residual QMV requires bfloat16 or float16")
    if autotune:
        from . import tuning

        tuning.ensure_dense_plan([weight], values.dtype)
    return dense_qmv(values, weight, residual)
