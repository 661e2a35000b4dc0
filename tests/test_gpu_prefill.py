"""Prefill affine GEMM on the GPU (M = 512 at Qwen2.5-1.5B shape, up
K=1536 N=8960 and down K=8960 N=1536).

Reference: fp32-accumulated ``x @ dequantize(w).T`` over the exact fp32 dequantized weights
(the oracle). Contract: tolerance_error <= 2e-3 (max-abs normalised, after the final output
rounding). The GEMM keeps dequantization exact (code-domain MFMA with per-group fp32 affine
terms), so in addition at least 98% (bf16) / 90% (f16) of the outputs must equal the correctly
rounded reference, which pins the tiling and indexing exactly.
"""

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


def reference(x, w, g, dtype):
    deq = O.dequantize(*w, g, 4, dtype)
    return (O.to_f32(x, dtype) @ deq.T).astype(np.float64)   # fp32 accumulation (BLAS)


def run_case(name, m, k, n, g=64, dtype="bf16", config_id=4):
    w = O.make_affine_weight(n, k, 4, g, config_id, 10, dtype)
    x = O.make_activations(m, k, config_id, dtype=dtype)
    ref = reference(x, w, g, dtype)
    aw = mt.AffineWeight.from_torch(*affine_to_torch(w, dtype), group_size=g) if g == 64 else None
    xt = act_to_torch(x, dtype)
    if aw is not None:
        y = mt.mlx_affine_matmul(xt, aw)
    else:
        y = mt.affine_matmul(xt, *affine_to_torch(w, dtype), group_size=g)
    got = torch_to_act(y, dtype)
    err = O.tolerance_error(got, ref, dtype)
    exact_frac = float(np.mean(O.to_f32(got, dtype) ==
                               O.to_f32(O.from_f32(ref.astype(np.float32), dtype), dtype)))
    print(f"[{name}] tolerance_error={err:.3e} exact_fraction={exact_frac:.4f}", flush=True)
    assert err <= 2e-3, (name, err)
    assert exact_frac >= (0.98 if dtype == "bf16" else 0.90), (name, exact_frac)


def test_prefill_up_config4():
    run_case("prefill up M=512 K=1536 N=8960", 512, 1536, 8960)


def test_prefill_down_config4():
    run_case("prefill down M=512 K=8960 N=1536", 512, 8960, 1536)


@pytest.mark.parametrize("m,k,n,g,dtype", [
    (33, 512, 96, 64, "bf16"),      # ragged rows and columns (partial 64 x 64 tiles)
    (200, 1024, 160, 128, "bf16"),  # group 128
    (130, 768, 256, 64, "f16"),
    (1, 256, 64, 64, "bf16"),
])
def test_prefill_shapes(m, k, n, g, dtype):
    run_case(f"prefill M={m} K={k} N={n} g{g} {dtype}", m, k, n, g, dtype, config_id=m + n)


def test_prefill_leading_dims():
    w = O.make_affine_weight(128, 256, 4, 64, 7, 10)
    x = O.make_activations(12, 256, 7)
    aw = mt.AffineWeight.from_torch(*affine_to_torch(w, "bf16"))
    flat = mt.mlx_affine_matmul(act_to_torch(x, "bf16"), aw)
    shaped = mt.mlx_affine_matmul(act_to_torch(x, "bf16").reshape(3, 4, 256), aw)
    assert tuple(shaped.shape) == (3, 4, 128)
    assert torch.equal(shaped.reshape(12, 128).view(torch.int16), flat.view(torch.int16))


# Every plan the library lists at a ragged shape, in both 16-bit types and both group sizes:
# partial output tiles in rows and columns for every tile width, split lengths that are not
# whole three-step iterations (the ring kernel runs its padding steps over zeros), and splits
# whose start falls inside a group of 128.
@pytest.mark.parametrize("g,dtype", [(64, "f16"), (128, "bf16")])
def test_every_prefill_plan_at_a_ragged_shape(g, dtype):
    from metile_amd import tuning

    m, k, n = 150, 1280, 480
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    w = O.make_affine_weight(n, k, 4, g, 21, 10, dtype)
    x = O.make_activations(m, k, 21, dtype=dtype)
    ref = reference(x, w, g, dtype)
    wt = affine_to_torch(w, dtype)
    xt = act_to_torch(x, dtype)
    cands = tuning.gemm_plan_candidates(m, k, n, g)
    assert {c.kernel for c in cands} == {"staged", "ring"}
    try:
        for plan in cands:
            print(f"[prefill ragged {dtype} g{g}] plan {plan}", flush=True)
            tuning.install_gemm_plan(m, k, n, g, tdt, plan)
            got = torch_to_act(mt.affine_matmul(xt, *wt, group_size=g), dtype)
            torch.cuda.synchronize()
            err = O.tolerance_error(got, ref, dtype)
            exact = float(np.mean(O.to_f32(got, dtype) ==
                                  O.to_f32(O.from_f32(ref.astype(np.float32), dtype), dtype)))
            assert err <= 2e-3 and exact >= (0.98 if dtype == "bf16" else 0.90), (plan, err, exact)
    finally:
        tuning.clear_plans()
