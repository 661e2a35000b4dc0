"""The native compositions (the reference's semantics: quantized matmul, then SwiGLU or the
residual add in the activation dtype) and the fidelity gates on the GPU: the kernels must pass
the reference tuner's gate against them (metile/backends/mlx_quantized.py:1256-1272,1297)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import metile_amd as mt
from oracle import affine as O
from tests.helpers import act_to_torch, affine_to_torch, torch_to_act

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)


@pytest.mark.parametrize("m,bits,g", [(1, 4, 64), (8, 4, 64), (3, 8, 64), (2, 8, 32)])
def test_swiglu_kernel_passes_gate_against_native(m, bits, g):
    gate = affine_to_torch(O.make_affine_weight(1024, 512, bits, g, 8, 10), "bf16")
    up = affine_to_torch(O.make_affine_weight(1024, 512, bits, g, 8, 12), "bf16")
    x = act_to_torch(O.make_activations(m, 512, 8), "bf16")
    kernel = mt.mlx_affine_swiglu(x, *gate, *up, bits=bits, group_size=g)
    native = mt.native_affine_swiglu(x, *gate, *up, bits=bits, group_size=g)
    assert mt.affine_swiglu_compatible(kernel, native)
    # the native path itself against the oracle's fp64 SwiGLU, with the same gate
    ref = O.affine_swiglu(O.make_activations(m, 512, 8),
                          O.make_affine_weight(1024, 512, bits, g, 8, 10),
                          O.make_affine_weight(1024, 512, bits, g, 8, 12), g, bits)
    ref_t = act_to_torch(O.from_f32(ref.astype(np.float32), "bf16"), "bf16")
    assert mt.affine_swiglu_compatible(native, ref_t)


def test_residual_and_matmul_natives():
    w = O.make_affine_weight(256, 1024, 4, 64, 9, 10)
    x = O.make_activations(5, 1024, 9)
    r = O.make_activations(5, 256, 9, tensor_id=3)
    wt = affine_to_torch(w, "bf16")
    xt, rt = act_to_torch(x, "bf16"), act_to_torch(r, "bf16")
    native = mt.native_affine_residual_qmv(xt, *wt, rt)
    kernel = mt.mlx_affine_residual_qmv(xt, *wt, rt)
    assert mt.affine_swiglu_compatible(kernel, native)
    aw = mt.AffineWeight.from_torch(*wt)
    xp = act_to_torch(O.make_activations(130, 1024, 9), "bf16")
    assert mt.accuracy_compatible(mt.mlx_affine_matmul(xp, aw), mt.native_affine_matmul(xp, aw))


def test_executors_gate_their_kernels_on_the_sample():
    gate = affine_to_torch(O.make_affine_weight(384, 256, 4, 64, 11, 10), "bf16")
    up = affine_to_torch(O.make_affine_weight(384, 256, 4, 64, 11, 12), "bf16")
    down = affine_to_torch(O.make_affine_weight(256, 384, 4, 64, 11, 14), "bf16")
    x = act_to_torch(O.make_activations(2, 256, 11), "bf16")
    r = act_to_torch(O.make_activations(2, 256, 11, tensor_id=3), "bf16")
    ex = mt.mlx_affine_mlp_executor(x, *gate, *up, *down, r)
    y = ex(x, r)
    # the executor is the two kernels in a row, bit for bit
    hidden = mt.mlx_affine_swiglu(x, *gate, *up)
    assert torch.equal(y, mt.mlx_affine_residual_qmv(hidden, *down, r))
    # the reference gates each stage against its native composition on that stage's input
    # (metile/backends/mlx_quantized.py:1786-1828): SwiGLU on x, the residual QMV on the
    # kernel's own hidden activations
    assert mt.affine_swiglu_compatible(hidden, mt.native_affine_swiglu(x, *gate, *up))
    assert mt.affine_swiglu_compatible(y, mt.native_affine_residual_qmv(hidden, *down, r))
    # end to end the two bf16 roundings of the hidden activations compound; the reference
    # gates no whole-MLP result, so the looser accuracy rule of its dense paths applies here
    want = mt.native_affine_residual_qmv(mt.native_affine_swiglu(x, *gate, *up), *down, r)
    assert mt.accuracy_compatible(y, want)
