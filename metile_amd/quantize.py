"""Affine group quantization of dense weights on the GPU, and the INT8 down-projection weight.

``affine_quantize`` turns a dense 16-bit ``[N, K]`` weight into the MLX affine format the
kernels read (``mx.quantize(weight, group_size, bits, mode="affine")``, the call in
``metile/backends/mlx_compressed_down.py:41-48``), with the gfx950 kernel behind
``mt_affine_quantize``. ``CompressedDownWeight`` mirrors ``MLXCompressedDownWeight``
(``metile/backends/mlx_compressed_down.py:21-83``): an affine INT8 output-major weight that
quantizes itself and applies ``quantized_matmul`` semantics when called.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .quantized import _DTYPES, _require_device, _stream_handle, affine_qmv


def affine_quantize(weight, *, group_size=64, bits=4):
    """``(w_q, scales, biases)`` of ``weight`` ``[N, K]`` (bfloat16 or float16) in the MLX affine
    format: ``w_q`` int32 words ``[N, K*bits/32]``, scales and biases ``[N, K/group_size]`` in
    ``weight``'s dtype. Per group the scale and bias make the extreme of larger magnitude exactly
    representable; codes are ``rint((w - bias) / scale)`` with the stored scale and bias."""
    _require_device(weight)
    if bits not in (4, 8):
        raise ValueError("affine quantization supports 4 and 8 bits")
    if group_size not in (32, 64, 128):
        raise ValueError("affine group size must be 32, 64, or 128")
    if weight.ndim != 2:
        raise ValueError("affine quantization expects a matrix")
    try:
        code = _DTYPES[weight.dtype]
    except KeyError:
        raise ValueError("weights must be bfloat16 or float16") from None
    n, k = weight.shape
    if k % group_size:
        raise ValueError("the input dimension must be a multiple of the group size")
    w = weight.contiguous()
    w_q = torch.empty(n, k * bits // 32, dtype=torch.int32, device=w.device)
    scales = torch.empty(n, k // group_size, dtype=w.dtype, device=w.device)
    biases = torch.empty_like(scales)
    _lib.check(_lib.lib().mt_affine_quantize(
        w.data_ptr(), w_q.data_ptr(), scales.data_ptr(), biases.data_ptr(), n, k, group_size,
        bits, code, _stream_handle(w.device)))
    return w_q, scales, biases


@dataclass(frozen=True)
class CompressedDownWeight:
    """An affine INT8 output-major weight (``MLXCompressedDownWeight``,
    ``metile/backends/mlx_compressed_down.py:21-83``). Only the ``affine8`` format is built;
    the reference's ``mxfp8`` format is a block-scaled format outside this build."""

    values: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    shape: tuple
    format: str
    group_size: int

    @classmethod
    def quantize(cls, weight, *, format="affine8", group_size=64):
        if weight.ndim != 2:
            raise ValueError("compressed down-projection weights must be matrices")
        if format == "affine8":
            if group_size not in {32, 64, 128}:
                raise ValueError("affine8 group size must be 32, 64, or 128")
            values, scales, biases = affine_quantize(weight, group_size=group_size, bits=8)
        elif format == "mxfp8":
            raise ValueError("the mxfp8 compressed down format is not built for gfx950")
        else:
            raise ValueError("compressed down format must be affine8 or mxfp8")
        return cls(values, scales, biases, tuple(weight.shape), format, group_size)

    @property
    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in (self.values, self.scales, self.biases))

    def __call__(self, values):
        """``values @ dequantize(weight).T`` (``mx.quantized_matmul`` semantics), any rows."""
        return affine_qmv(values, self.values, self.scales, self.biases,
                          group_size=self.group_size, bits=8)
