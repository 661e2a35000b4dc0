"""The reference's argument guards, reproduced with the same exception types and messages
(metile/backends/mlx_quantized.py:1550-1568,1659-1670). CPU only: guards run before any
device work."""

from __future__ import annotations

import pytest
import torch

import metile_amd as mt


def _affine(n, k, bits=4, g=64, dtype=torch.bfloat16):
    w = torch.zeros(n, k * bits // 32, dtype=torch.int32)
    s = torch.zeros(n, k // g, dtype=dtype)
    return w, s, s.clone()


def test_residual_qmv_requires_4bit_group64():
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    w, s, b = _affine(64, 128, bits=8)
    with pytest.raises(ValueError, match="4-bit weights with group size 64"):
        mt.mlx_affine_residual_qmv(x, w, s, b, torch.zeros(1, 64, dtype=torch.bfloat16),
                                   bits=8)


def test_residual_qmv_requires_biases():
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    w, s, _ = _affine(64, 128)
    with pytest.raises(ValueError, match="requires affine quantization biases"):
        mt.mlx_affine_residual_qmv(x, w, s, None, torch.zeros(1, 64, dtype=torch.bfloat16))


def test_residual_qmv_rejects_incompatible_parameters():
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    w, s, b = _affine(64, 256)
    with pytest.raises(ValueError, match="incompatible quantization parameters"):
        mt.mlx_affine_residual_qmv(x, w, s, b, torch.zeros(1, 64, dtype=torch.bfloat16))


def test_residual_qmv_rejects_dtype_mismatch():
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    w, s, b = _affine(64, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="must match the input dtype"):
        mt.mlx_affine_residual_qmv(x, w, s, b, torch.zeros(1, 64, dtype=torch.bfloat16))


def test_residual_qmv_rejects_residual_shape():
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    w, s, b = _affine(64, 128)
    with pytest.raises(ValueError, match="residual must match"):
        mt.mlx_affine_residual_qmv(x, w, s, b, torch.zeros(1, 32, dtype=torch.bfloat16))


@pytest.mark.parametrize("bits,g", [(4, 32), (4, 128), (8, 256), (2, 64)])
def test_swiglu_rejects_unsupported_formats(bits, g):
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    w, s, b = _affine(64, 256, bits=4, g=64)
    with pytest.raises(ValueError, match="4-bit group-64 or 8-bit group-32/64/128"):
        mt.mlx_affine_swiglu(x, w, s, b, w, s, b, bits=bits, group_size=g)


def test_swiglu_requires_biases_and_matching_pairs():
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    w, s, b = _affine(64, 256)
    with pytest.raises(ValueError, match="requires affine quantization biases"):
        mt.mlx_affine_swiglu(x, w, s, b, w, s, None)
    w2, s2, b2 = _affine(32, 256)
    with pytest.raises(ValueError, match="matching gate/up"):
        mt.mlx_affine_swiglu(x, w, s, b, w2, s2, b2)


def test_mlp_executor_applies_residual_guard_to_down():
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    gw, gs, gb = _affine(128, 256, bits=8)
    dw, ds, db = _affine(256, 128, bits=8)
    with pytest.raises(ValueError, match="4-bit weights with group size 64"):
        mt.mlx_affine_mlp_executor(x, gw, gs, gb, gw, gs, gb, dw, ds, db,
                                   torch.zeros(1, 256, dtype=torch.bfloat16), bits=8)


def test_operators_reject_host_tensors():
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    w, s, b = _affine(64, 128)
    with pytest.raises(ValueError, match="ROCm device tensors"):
        mt.affine_qmv(x, w, s, b)
