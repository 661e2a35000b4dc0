"""Every listed prefill-GEMM plan and every listed dense plan at seeded random shapes, on the GPU
through the C ABI.

* GEMM (``mt_affine_gemm_plan_candidates``), 16 shapes and 4 edge shapes: M from 1 to 300 rows,
  K a multiple of 64 up to 2048, N a multiple of 32 up to 1536, groups of 64 and 128, bf16 and
  f16. Every plan is held to the contract against the fp64 product of the activations and the
  exactly dequantized weights: ``tolerance_error`` <= 2e-3 and >= 98% (bf16) / 90% (f16) of
  outputs equal to the correctly rounded value.
* Dense (``mt_dense_qmv_plan_candidates``, K splits keyed by (K, N)), 16 shapes and 2 edge
  shapes: M from 1 to 130 rows, fused SwiGLU and the projection with or without the residual,
  bf16 and f16. Every plan is held to the typed-epilogue contract of ``test_gpu_dense.py``
  (>= 99% bit-exact, within 3 operand ulps, ``tolerance_error`` <= 2e-3 after the reference's
  own rounding budget), and rows of the batch are bit-identical to the same rows run alone under
  the same plan.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import metile_amd as mt
from metile_amd import tuning
from oracle import affine as O
from tests.helpers import act_to_torch, affine_to_torch, torch_to_act
from tests.test_gpu_dense import check_typed, dots

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _gemm_shapes():
    rng = np.random.RandomState(4242)
    out = []
    for _ in range(16):
        g = int(rng.choice([64, 128]))
        k = int(rng.randint(1, 17)) * 128 if g == 128 else int(rng.randint(1, 33)) * 64
        n = int(rng.randint(1, 49)) * 32
        m = int(rng.randint(1, 301))
        dtype = "f16" if rng.randint(3) == 0 else "bf16"
        out.append((m, k, n, g, dtype))
    # edges: one row, one K step, one 128 x 128 tile exactly, rows just past a tile
    out += [(1, 512, 256, 64, "bf16"), (64, 64, 32, 64, "bf16"), (128, 1024, 128, 128, "bf16"),
            (129, 640, 96, 64, "f16")]
    return out


def _dense_shapes():
    rng = np.random.RandomState(777)
    out = []
    for _ in range(16):
        k = int(rng.randint(1, 33)) * 64
        n = int(rng.randint(1, 49)) * 32
        m = int(rng.choice([1, 2, 3, 8, 17, 32, 33, 64, 65, 100, 128, 130]))
        nproj = int(rng.choice([1, 2]))
        residual = nproj == 1 and bool(rng.randint(2))
        dtype = "f16" if rng.randint(3) == 0 else "bf16"
        out.append((m, k, n, nproj, residual, dtype))
    out += [(1, 64, 32, 2, False, "bf16"), (130, 64, 32, 1, True, "bf16")]
    return out


GEMM_SWEEP = _gemm_shapes()
DENSE_SWEEP = _dense_shapes()


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


@pytest.mark.parametrize("shape", GEMM_SWEEP, ids=lambda s: "x".join(map(str, s)))
def test_every_gemm_plan_at_random_shapes(shape):
    m, k, n, g, dtype = shape
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    w = O.make_affine_weight(n, k, 4, g, 41, 10, dtype)
    x = O.make_activations(m, k, 41, dtype=dtype)
    wf = O.dequantize(*w, g, 4, dtype).astype(np.float64)
    ref = O.to_f32(x, dtype).astype(np.float64) @ wf.T
    want = O.to_f32(O.from_f32(ref.astype(np.float32), dtype), dtype)
    wt = affine_to_torch(w, dtype)
    xt = act_to_torch(x, dtype)
    min_exact = 0.98 if dtype == "bf16" else 0.90
    cands = tuning.gemm_plan_candidates(m, k, n, g)
    assert tuning.gemm_plan(m, k, n, g, tdt) in cands
    for plan in cands:
        print(f"[gemm {shape}] plan {plan}", flush=True)
        tuning.install_gemm_plan(m, k, n, g, tdt, plan)
        y = torch_to_act(mt.affine_matmul(xt, *wt, group_size=g, bits=4), dtype)
        torch.cuda.synchronize()
        err = O.tolerance_error(y, ref, dtype)
        exact = np.mean(O.to_f32(y, dtype) == want)
        assert err <= TOL and exact >= min_exact, (plan, err, exact)
    print(f"[gemm {shape}] {len(cands)} plans", flush=True)


@pytest.mark.parametrize("shape", DENSE_SWEEP, ids=lambda s: "x".join(map(str, s)))
def test_every_dense_plan_at_random_shapes(shape):
    m, k, n, nproj, residual, dtype = shape
    x = O.make_activations(m, k, 43, dtype=dtype)
    ws = [O.make_dense_weight(n, k, 43, 10 + p, dtype=dtype) for p in range(nproj)]
    r = O.make_activations(m, n, 43, tensor_id=3, dtype=dtype) if residual else None
    if nproj == 2:
        want = O.dense_swiglu(x, ws[0], ws[1], dtype=dtype)
        scale = dots(x, ws[0], dtype) * dots(x, ws[1], dtype)
        exact = O.dense_swiglu_exact(x, ws[0], ws[1], dtype=dtype)
    else:
        want = O.dense_residual_qmv(x, ws[0], r, dtype=dtype)
        scale = np.abs(dots(x, ws[0], dtype))
        if r is not None:
            scale = np.maximum(scale, np.abs(O.to_f32(r, dtype)))
        exact = O.dense_residual_exact(x, ws[0], r, dtype=dtype)
    xt = act_to_torch(x, dtype)
    wts = [act_to_torch(w, dtype) for w in ws]
    rt = None if r is None else act_to_torch(r, dtype)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16

    def run(xv, rv):
        if nproj == 2:
            return mt.dense_swiglu(xv, wts[0], wts[1])
        return mt.dense_qmv(xv, wts[0], rv)

    # short K lists no split plan: the planner's (one split) is then the only plan
    plans = tuning.dense_plan_candidates(k, n, nproj) or [None]
    try:
        for plan in plans:
            print(f"[dense {shape}] plan {plan}", flush=True)
            tuning.install_dense_plan(k, n, nproj, tdt, plan)
            batch = run(xt, rt)
            check_typed(f"dense {shape} {plan}", torch_to_act(batch, dtype), want, scale, exact,
                        dtype, ulps=3.0)
            for row in sorted({0, m // 2, m - 1}):
                one = run(xt[row:row + 1], None if rt is None else rt[row:row + 1])
                assert torch.equal(one.view(torch.int16), batch[row:row + 1].view(torch.int16)), \
                    (plan, row)
    finally:
        tuning.install_dense_plan(k, n, nproj, tdt, None)
