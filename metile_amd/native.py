"""The reference's native compositions (its semantics), on torch tensors of a ROCm device.

The reference checks its kernels against ``mx.quantized_matmul`` compositions:
``_native_affine_residual_qmv`` (``metile/backends/mlx_quantized.py:834-855``),
``_native_affine_swiglu`` (``:883-917``) and ``_native_affine_matmul``
(``metile/backends/mlx_affine.py:142-154``). Here the quantized matmul is the exact fp32
dequantization (``affine_dequantize``, a gfx950 kernel) followed by an fp32 torch matmul,
rounded to the activation dtype; SwiGLU and the residual add then run in that dtype, as the
MLX compositions do. These are comparison paths for the fidelity gates, not the product path.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .quantized import AffineWeight, affine_dequantize


def _quantized_matmul(values, weight, scales, biases, group_size, bits):
    w = affine_dequantize(weight, scales, biases, group_size=group_size, bits=bits)  # [N, K]
    k = values.shape[-1]
    y = values.reshape(-1, k).float() @ w.t()
    return y.to(values.dtype).reshape(*values.shape[:-1], w.shape[0])


def native_affine_residual_qmv(values, weight, scales, biases, residual, *, group_size=64,
                               bits=4):
    """``quantized_matmul(values, weight) + residual`` (``mlx_quantized.py:834-855``)."""
    projected = _quantized_matmul(values, weight, scales, biases, group_size, bits)
    return projected if residual is None else projected + residual


def native_affine_swiglu(values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                         up_biases, *, group_size=64, bits=4):
    """``silu(gate) * up`` over two quantized matmuls (``mlx_quantized.py:883-917``)."""
    gate = _quantized_matmul(values, gate_weight, gate_scales, gate_biases, group_size, bits)
    up = _quantized_matmul(values, up_weight, up_scales, up_biases, group_size, bits)
    return F.silu(gate) * up


def native_affine_matmul(values, weight: AffineWeight):
    """``quantized_matmul`` with an ``AffineWeight`` (``metile/backends/mlx_affine.py:142-154``)."""
    return _quantized_matmul(values, weight.native_weight, weight.native_scales,
                             weight.native_biases, weight.group_size, weight.bits)
