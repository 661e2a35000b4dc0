"""The reference tuner's fidelity gates (CPU): restating
metile/backends/mlx_quantized.py:1256-1272 and metile/backends/mlx_affine.py:273-278."""

from __future__ import annotations

import pytest
import torch

import metile_amd as mt


def _ref(n=4096, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, generator=g).to(torch.bfloat16)


def test_swiglu_gate_accepts_identical_and_rounding_noise():
    ref = _ref()
    assert mt.affine_swiglu_compatible(ref.clone(), ref)
    # every tenth element one bf16 ulp up (at most 2^-7 of its magnitude): RMS ratio about
    # 0.001, peak ratio below 2^-7
    bits = ref.view(torch.int16).clone()
    bits[::10] += 1
    assert mt.affine_swiglu_compatible(bits.view(torch.bfloat16), ref)


def test_swiglu_gate_rejects_rms_peak_nonfinite_shape_dtype():
    ref = _ref()
    # a uniform 1% error: RMS ratio 0.01 > 0.005
    assert not mt.affine_swiglu_compatible((ref.float() * 1.01).to(torch.bfloat16), ref)
    # one large outlier: peak ratio above 0.01 while the RMS ratio stays small
    bad = ref.clone()
    i = int(torch.argmax(ref.float().abs()))
    bad[i] = (ref[i].float() * 1.05).to(torch.bfloat16)
    assert not mt.affine_swiglu_compatible(bad, ref)
    nan = ref.clone()
    nan[3] = float("nan")
    assert not mt.affine_swiglu_compatible(nan, ref)
    assert not mt.affine_swiglu_compatible(ref.reshape(64, 64), ref)
    assert not mt.affine_swiglu_compatible(ref.to(torch.float16), ref)


def test_swiglu_gate_floors_tiny_references():
    ref = torch.zeros(16, dtype=torch.bfloat16)
    assert mt.affine_swiglu_compatible(torch.full((16,), 1e-9).to(torch.bfloat16), ref)
    assert not mt.affine_swiglu_compatible(torch.full((16,), 1e-7).to(torch.bfloat16), ref)


def test_accuracy_gate():
    ref = torch.tensor([0.0, 1.0, -3.0])
    assert mt.accuracy_compatible(ref + 0.079, ref)          # bound 0.02 + 0.02 * 3 = 0.08
    assert not mt.accuracy_compatible(ref + 0.081, ref)
    assert mt.accuracy_compatible(torch.zeros(3) + 0.0199, torch.zeros(3))
    assert not mt.accuracy_compatible(torch.zeros(3) + 0.0201, torch.zeros(3))


def test_gates_raise_on_empty_like_the_reference():
    with pytest.raises(RuntimeError):
        mt.accuracy_compatible(torch.zeros(0), torch.zeros(0))
