"""The 4x4x4-MFMA GEMV kernel (``MT_QMV_GEMV4``) on the GPU, through the C ABI, against the oracle.

Every case installs the kernel's plans for its shape and checks the result against the oracle's
(``tolerance_error`` <= 2e-3 and >= 98% (bf16) / 90% (f16) of outputs equal to the correctly
rounded reference), over MLX codes and over repacked codes (bit-identical), at 1 to 4 rows, bf16
and f16, groups of 32, 64 and 128, one and two projections (with and without the residual), K a
whole number of 512-wide rounds or not (the last round's blocks past K read zeros), and every wave
count and column-group count the plan list offers (one to four rounds per wave, waves with no
round of their own, 4 to 16 columns per workgroup).
"""

from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

import metile_amd as mt
from metile_amd import tuning
from oracle import affine as O
from tests.helpers import act_to_torch, affine_to_torch, torch_to_act

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)


@pytest.fixture(autouse=True)
def _clean_plans():
    tuning.clear_plans()
    yield
    tuning.clear_plans()


@functools.lru_cache(maxsize=4)
def _case(k, n, g, nproj, residual, dtype, rows):
    weights = [O.make_affine_weight(n, k, 4, g, 23, 10 + 2 * p, dtype) for p in range(nproj)]
    x = O.make_activations(rows, k, 23, dtype=dtype)
    res = O.make_activations(rows, n, 23, tensor_id=3, dtype=dtype) if residual else None
    if nproj == 2:
        ref = O.affine_swiglu(x, weights[0], weights[1], g, 4, dtype=dtype)
    else:
        ref = O.affine_qmv(x, *weights[0], g, 4, residual=res, dtype=dtype)
    return weights, x, res, ref


def _plans(rows, k, n, g, nproj):
    plans = [p for p in tuning.qmv_plan_candidates(rows, k, n, g, 4, nproj) if p.kernel == "gemv4"]
    assert {n // p.strips // 4 for p in plans} <= {1, 2, 4} and plans
    return plans


def _run(rows, k, n, g, nproj, residual, dtype, plans=None):
    weights, x, res, ref = _case(k, n, g, nproj, residual, dtype, rows)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    xt = act_to_torch(x, dtype)
    rt = None if res is None else act_to_torch(res, dtype)
    mlx = [affine_to_torch(w, dtype) for w in weights]
    packed = [(mt.affine_repack(w, bits=4), s, b) for (w, s, b) in mlx]

    def run(ts):
        if nproj == 2:
            return mt.affine_swiglu(xt, *ts[0], *ts[1], group_size=g, bits=4)
        return mt.affine_qmv(xt, *ts[0], group_size=g, bits=4, residual=rt)

    min_exact = 0.98 if dtype == "bf16" else 0.90
    for plan in plans if plans is not None else _plans(rows, k, n, g, nproj):
        print(f"[{rows}x{k}x{n} g{g} p{nproj} {dtype}] plan {plan}", flush=True)
        tuning.install_qmv_plan(rows, k, n, g, 4, nproj, tdt, plan)
        assert tuning.qmv_plan(rows, k, n, g, 4, nproj, tdt) == plan
        a, b = run(mlx), run(packed)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), plan
        y = torch_to_act(a, dtype)
        err = O.tolerance_error(y, ref, dtype)
        exact = np.mean(O.to_f32(y, dtype) == O.to_f32(O.from_f32(ref.astype(np.float32), dtype),
                                                       dtype))
        assert err <= TOL and exact >= min_exact, (plan, err, exact)


@pytest.mark.parametrize("rows", [1, 2, 3, 4])
def test_swiglu_config1_shape(rows):
    # gate/up at the headline shape: K = 1536 is three rounds
    _run(rows, 1536, 8960, 64, 2, False, "bf16")


@pytest.mark.parametrize("rows", [1, 4])
def test_down_residual_config1_shape(rows):
    # K = 8960: 17.5 rounds, the last half past K; five to eight waves
    _run(rows, 8960, 1536, 64, 1, True, "bf16")


@pytest.mark.parametrize("g,dtype", [(32, "bf16"), (128, "f16"), (64, "f16")])
def test_groups_and_dtypes(g, dtype):
    _run(3, 2048, 512, g, 1, False, dtype)
    _run(2, 1024, 256, g, 2, False, dtype)


def test_short_k_and_one_round():
    # K below one round (the blocks past K read zeros) and exactly one round
    _run(2, 256, 128, 64, 1, True, "bf16")
    _run(1, 512, 96, 32, 2, False, "bf16")


def test_rows_are_independent_of_the_batch():
    # a row's output is the same bits alone and inside a four-row dispatch (MFMA rows do not mix)
    k, n, g = 1536, 1024, 64
    weights, x, _, _ = _case(k, n, g, 1, False, "bf16", 4)
    ts = affine_to_torch(weights[0], "bf16")
    xt = act_to_torch(x, "bf16")
    plan = _plans(4, k, n, g, 1)[0]
    tuning.install_qmv_plan(4, k, n, g, 4, 1, torch.bfloat16, plan)
    tuning.install_qmv_plan(1, k, n, g, 4, 1, torch.bfloat16, plan)
    full = mt.affine_qmv(xt, *ts, group_size=g, bits=4)
    for r in range(4):
        one = mt.affine_qmv(xt[r:r + 1].contiguous(), *ts, group_size=g, bits=4)
        assert torch.equal(one.view(torch.int16), full[r:r + 1].view(torch.int16)), r

