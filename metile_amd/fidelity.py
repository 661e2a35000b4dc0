"""Fidelity gates of the reference tuner, on torch tensors.

The reference accepts a kernel candidate only if its output passes one of these checks against
the native MLX composition on the same sample inputs:

* ``affine_swiglu_compatible`` restates ``_affine_swiglu_compatible``
  (``metile/backends/mlx_quantized.py:1256-1272``): same shape and dtype, every value finite,
  RMS of the difference at most 0.005 of the reference's RMS and the largest difference at most
  0.01 of the reference's largest magnitude (both denominators floored at 1e-6), all in fp32.
  The reference applies it to affine SwiGLU and residual-QMV candidates
  (``metile/backends/mlx_quantized.py:1297``).
* ``accuracy_compatible`` restates ``_accuracy_compatible``
  (``metile/backends/mlx_affine.py:273-278``, the same rule in ``mlx_dense.py:239-244`` and
  ``mlx_dense_swiglu.py:297-302``): largest absolute difference at most
  ``0.02 + 0.02 * max|reference|``. The difference is taken in fp32 here (MLX subtracts in the
  arrays' own dtype; at these thresholds the two agree).

Like the reference's reductions, both raise on empty tensors.
"""

from __future__ import annotations

import torch


def affine_swiglu_compatible(result: torch.Tensor, reference: torch.Tensor) -> bool:
    if result.shape != reference.shape or result.dtype != reference.dtype:
        return False
    r = result.float()
    ref = reference.float()
    diff = r - ref
    reference_rms = torch.sqrt(torch.mean(ref * ref))
    difference_rms = torch.sqrt(torch.mean(diff * diff))
    reference_peak = torch.max(torch.abs(ref))
    difference_peak = torch.max(torch.abs(diff))
    finite = bool(torch.isfinite(r).all())
    floor = torch.tensor(1e-6, dtype=torch.float32, device=r.device)
    normalized_rms = float(difference_rms / torch.maximum(reference_rms, floor))
    normalized_peak = float(difference_peak / torch.maximum(reference_peak, floor))
    return finite and normalized_rms <= 0.005 and normalized_peak <= 0.01


def accuracy_compatible(actual: torch.Tensor, reference: torch.Tensor) -> bool:
    maximum_error = float(torch.max(torch.abs(actual.float() - reference.float())))
    reference_scale = float(torch.max(torch.abs(reference.float())))
    return maximum_error <= 0.02 + 0.02 * reference_scale
