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


# ---- dense (metile/backends/mlx_dense_swiglu.py:424-447, mlx_dense_residual.py:276-288) ----


def test_dense_weight_validation():
    with pytest.raises(ValueError, match="shape \\[output, input\\]"):
        mt.DenseWeight.from_torch(torch.zeros(4, dtype=torch.bfloat16))
    with pytest.raises(TypeError, match="bfloat16 or float16"):
        mt.DenseWeight.from_torch(torch.zeros(4, 4, dtype=torch.float32))
    assert mt.DenseWeight.from_torch(torch.zeros(64, 128, dtype=torch.bfloat16)).shape == (128, 64)


def test_dense_swiglu_guards():
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    g = mt.DenseWeight.from_torch(torch.zeros(64, 128, dtype=torch.bfloat16))
    with pytest.raises(TypeError, match="must be DenseWeight"):
        mt.mlx_dense_swiglu(x, g.native_weight, g)
    u2 = mt.DenseWeight.from_torch(torch.zeros(32, 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="matching shapes"):
        mt.mlx_dense_swiglu(x, g, u2)
    with pytest.raises(ValueError, match="values\\[..., K\\]"):
        mt.mlx_dense_swiglu(torch.zeros(2, 64, dtype=torch.bfloat16), g, g)
    with pytest.raises(TypeError, match="matching activation and weight dtypes"):
        mt.mlx_dense_swiglu(x.half(), g, g)
    with pytest.raises(ValueError, match="paired dense SwiGLU weight"):
        mt.mlx_dense_swiglu(x, g, g, paired_weight=torch.zeros(64, 128, dtype=torch.bfloat16))


def test_dense_residual_guards():
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    w = torch.zeros(64, 128, dtype=torch.bfloat16)
    r = torch.zeros(2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="rank-compatible"):
        mt.mlx_dense_residual_qmv(x, w, r[0])
    with pytest.raises(ValueError, match="input features must match"):
        mt.mlx_dense_residual_qmv(x, w[:, :64], r)
    with pytest.raises(ValueError, match="residual shape"):
        mt.mlx_dense_residual_qmv(x, w, torch.zeros(2, 32, dtype=torch.bfloat16))
    with pytest.raises(TypeError, match="matching input dtypes"):
        mt.mlx_dense_residual_qmv(x, w.half(), r)


# ---- prefill (metile/backends/mlx_affine.py:80-114,359-366) -------------------------------


def test_affine_weight_requires_4bit_group64():
    w, s, b = _affine(64, 128, bits=8)
    with pytest.raises(ValueError, match="group size 64 and 4 bits"):
        mt.AffineWeight.from_torch(w, s, b, bits=8)
    w, s, b = _affine(64, 128)
    assert mt.AffineWeight.from_torch(w, s, b).shape == (128, 64)


def test_affine_matmul_guards():
    w, s, b = _affine(64, 128)
    aw = mt.AffineWeight.from_torch(w, s, b)
    with pytest.raises(TypeError, match="AffineWeight"):
        mt.mlx_affine_matmul(torch.zeros(2, 128, dtype=torch.bfloat16), w)
    with pytest.raises(ValueError, match="values\\[..., K\\]"):
        mt.mlx_affine_matmul(torch.zeros(2, 64, dtype=torch.bfloat16), aw)
    with pytest.raises(TypeError, match="float16 or bfloat16"):
        mt.mlx_affine_matmul(torch.zeros(2, 128, dtype=torch.float32), aw)


def test_repack_guards():
    """repack_mlx_affine_weight's guards (metile/backends/mlx_quantized.py:765-767)."""
    w, s, b = _affine(64, 128)
    with pytest.raises(ValueError, match="requires affine biases"):
        mt.repack_mlx_affine_weight(w, s, None)
    with pytest.raises(ValueError, match="matching two-dimensional parameters"):
        mt.repack_mlx_affine_weight(w[0], s, b)
    with pytest.raises(ValueError, match="matching two-dimensional parameters"):
        mt.repack_mlx_affine_weight(w, s, b[:, :1])


def test_nax_entries_validate_schedule_and_layout():
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    w, s, b = _affine(64, 128)
    packed = torch.zeros(2, 64, 8, dtype=torch.int32)
    with pytest.raises(ValueError, match="unsupported affine QMV schedule"):
        mt.mlx_affine_qmv_nax(x, packed, s, b, output_features=64, block=48)
    with pytest.raises(ValueError, match="repacked weights"):
        mt.mlx_affine_qmv_nax(x, w, s, b, output_features=64)
    with pytest.raises(ValueError, match="repacked weights"):
        mt.mlx_affine_swiglu_qmv_nax(x, packed, s, b, packed, s, b, output_features=32)


def test_mixed_code_layouts_are_rejected():
    # gate and up share one layout; the down projection may take the other (checked on the GPU)
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    w, s, b = _affine(256, 128)
    packed = torch.zeros(2, 256, 8, dtype=torch.int32)
    dw, ds, db = _affine(128, 256)
    with pytest.raises(ValueError):
        mt.affine_swiglu(x, w, s, b, packed, s, b)
    with pytest.raises(ValueError, match="gate and up weights must share one code layout"):
        mt.affine_mlp(x, (w, s, b), (packed, s, b), (dw, ds, db))


def test_dequantize_validates_scale_and_code_shapes():
    """Scales and biases must be [N, K / group_size] for the codes given, or the kernel would
    index past them."""
    w, s, b = _affine(64, 256)
    with pytest.raises(ValueError, match="requires biases"):
        mt.affine_dequantize(w, s, None)
    with pytest.raises(ValueError, match="incompatible quantization parameters"):
        mt.affine_dequantize(w, s, b, group_size=32)  # scales hold 4 groups, 8 needed
    with pytest.raises(ValueError, match="incompatible quantization parameters"):
        mt.affine_dequantize(w, s, b[:, :2])
    with pytest.raises(ValueError, match="incompatible quantization parameters"):
        mt.affine_dequantize(w[:32], s, b)
    with pytest.raises(ValueError, match="two-dimensional"):
        mt.affine_dequantize(w[0], s, b)
    with pytest.raises(ValueError, match="4- and 8-bit"):
        mt.affine_dequantize(w, s, b, bits=3)
    with pytest.raises(ValueError, match="ROCm device tensors"):
        mt.affine_dequantize(w, s, b)  # valid shapes, host tensors


def test_bound_mlp_checks_its_weights_once_on_the_host():
    """``BoundMlp`` runs the MLP's weight checks at construction (no device work)."""
    import torch

    from metile_amd.quantized import BoundMlp

    h, i = 128, 256
    w = torch.zeros(i, h // 8, dtype=torch.int32)
    s = torch.zeros(i, h // 64, dtype=torch.bfloat16)
    dw = torch.zeros(h, i // 8, dtype=torch.int32)
    ds = torch.zeros(h, i // 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm device"):
        BoundMlp((w, s, s), (w, s, s), (dw, ds, ds))
