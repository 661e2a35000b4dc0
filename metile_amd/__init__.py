"""metile_amd — MI355X (gfx950) kernels for meTile's quantized-projection hot path.

Affine 4/8-bit quantized QMV, fused SwiGLU, the quantized MLP and dense 16-bit small-batch
projections, written as hand-written HIP kernels behind a C ABI (``include/metile_amd.h``) and
exposed here on torch tensors with the reference's call surface
(``metile/backends/mlx_quantized.py``), with the reference tuner's fidelity gates and native
compositions for checking kernels against its semantics.
"""

from ._lib import MetileError, version
from .dense import DenseWeight, dense_qmv, dense_swiglu, mlx_dense_residual_qmv, mlx_dense_swiglu
from .fidelity import accuracy_compatible, affine_swiglu_compatible
from .model import (
    QuantizedLinear,
    patch_graph_fusion,
    patch_quantized_mlp,
    quantize_mlp,
    restore_patches,
)
from .native import native_affine_matmul, native_affine_residual_qmv, native_affine_swiglu
from .quantize import CompressedDownWeight, affine_quantize
from .quantized import (
    AffineWeight,
    affine_dequantize,
    affine_matmul,
    affine_mlp,
    affine_qmv,
    affine_repack,
    affine_swiglu,
    mlx_affine_matmul,
    mlx_affine_matmul_dispatches,
    mlx_affine_mlp_executor,
    mlx_affine_qmv,
    mlx_affine_qmv_nax,
    mlx_affine_residual_qmv,
    mlx_affine_residual_qmv_dispatches,
    mlx_affine_swiglu,
    mlx_affine_swiglu_dispatches,
    mlx_affine_swiglu_executor,
    mlx_affine_swiglu_qmv,
    mlx_affine_swiglu_qmv_nax,
    repack_mlx_affine_weight,
)

__all__ = [
    "AffineWeight",
    "CompressedDownWeight",
    "QuantizedLinear",
    "affine_quantize",
    "patch_graph_fusion",
    "patch_quantized_mlp",
    "quantize_mlp",
    "restore_patches",
    "DenseWeight",
    "MetileError",
    "accuracy_compatible",
    "affine_swiglu_compatible",
    "native_affine_matmul",
    "native_affine_residual_qmv",
    "native_affine_swiglu",
    "dense_qmv",
    "dense_swiglu",
    "mlx_dense_residual_qmv",
    "mlx_dense_swiglu",
    "affine_dequantize",
    "affine_matmul",
    "affine_mlp",
    "affine_qmv",
    "affine_repack",
    "affine_swiglu",
    "mlx_affine_matmul",
    "mlx_affine_matmul_dispatches",
    "mlx_affine_mlp_executor",
    "mlx_affine_qmv",
    "mlx_affine_qmv_nax",
    "mlx_affine_residual_qmv",
    "mlx_affine_residual_qmv_dispatches",
    "mlx_affine_swiglu",
    "mlx_affine_swiglu_dispatches",
    "mlx_affine_swiglu_executor",
    "mlx_affine_swiglu_qmv",
    "mlx_affine_swiglu_qmv_nax",
    "repack_mlx_affine_weight",
    "version",
]
