"""The GEMV plans of the small-row projections (up to 4 rows, no K split) on the GPU.

Every GEMV plan (2, 4 or 8 columns per column group, 1 to 8 waves, both workgroup orders) is
installed in turn and run
through the C ABI at 1 to 4 rows, bf16 and f16, 4 and 8 bits, groups of 32 to 128, with and
without the residual, at K shorter than one pass of the workgroup's lanes and at K that leaves
a ragged last pass:

* results are within the kernels' tolerance of the oracle (float64 sums, one rounding);
* the kernels over MLX codes and over repacked codes agree bit for bit;
* a row's result does not depend on how many rows the dispatch holds (rows 0 and 1 of a
  four-row dispatch equal the one- and two-row dispatches bit for bit) under the same plan.

Biases are drawn independently of the scales here (the benchmark recipe ties them as
bias = -zero * scale), so a mix-up of the two or of their group index changes the result.
"""

from __future__ import annotations

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


def _weight(n, k, bits, g, seed, tensor, dtype):
    w_q, scales, _ = O.make_affine_weight(n, k, bits, g, seed, tensor, dtype)
    r = O.rng(seed, tensor + 7)
    biases = O.from_f32(r.standard_normal((n, k // g), dtype=np.float32) * np.float32(0.01),
                        dtype)
    return w_q, scales, biases


CASES = [  # (K, N, group, bits, dtype, nproj, residual)
    (8960, 1536, 64, 4, "bf16", 1, True),    # the down projection: 280 chunks per column
    (8960, 1536, 64, 4, "f16", 1, False),
    (1536, 8960, 64, 4, "bf16", 2, False),   # the gate/up shape: 48 chunks, most lanes idle
    (1536, 8960, 128, 4, "f16", 2, False),
    (1536, 8960, 64, 4, "bf16", 1, True),    # config 0: one projection, column groups
    (1536, 8960, 64, 4, "f16", 1, False),
    (4864, 896, 32, 8, "bf16", 1, True),     # 8 bits, groups of 32
    (1024, 1536, 64, 8, "f16", 2, False),
    (2624, 640, 32, 4, "bf16", 1, False),    # 82 chunks: ragged last pass at every width
    (256, 96, 128, 8, "f16", 1, True),       # 16 chunks, shorter than any pass
    (1024, 1536, 64, 4, "bf16", 2, False),   # 32 chunks: two column groups per wave
    (512, 640, 64, 8, "f16", 1, True),       # 32 chunks at 8 bits
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_gemv_plans_match_the_oracle_at_every_row_count(case):
    k, n, g, bits, dtype, nproj, residual = case
    seed = k + n + bits
    weights = [_weight(n, k, bits, g, seed, 10 + 3 * p, dtype) for p in range(nproj)]
    x = O.make_activations(4, k, seed, dtype=dtype)
    res = O.make_activations(4, n, seed, tensor_id=3, dtype=dtype) if residual else None
    if nproj == 2:
        ref = O.affine_swiglu(x, weights[0], weights[1], g, bits, dtype=dtype)
    else:
        ref = O.affine_qmv(x, *weights[0], g, bits, residual=res, dtype=dtype)
    xt = act_to_torch(x, dtype)
    rt = None if res is None else act_to_torch(res, dtype)
    mlx = [affine_to_torch(w, dtype) for w in weights]
    packed = [(mt.affine_repack(w, bits=bits), s, b) for (w, s, b) in mlx]
    tdt = xt.dtype

    def run(ts, rows):
        if nproj == 2:
            return mt.affine_swiglu(xt[:rows], *ts[0], *ts[1], group_size=g, bits=bits)
        r = None if rt is None else rt[:rows]
        return mt.affine_qmv(xt[:rows], *ts[0], group_size=g, bits=bits, residual=r)

    chunks = k * bits // 128

    def groups(w):  # column groups per workgroup
        if chunks <= 64:  # whole groups in every wave
            return w * (64 // chunks if chunks % 16 == 0 else 1)
        return 64 * w // chunks if chunks <= 64 * w and chunks % 16 == 0 else 1

    plans = [p for p in tuning.qmv_plan_candidates(1, k, n, g, bits, nproj) if p.kernel == "gemv"]
    # the listed wave counts, and the extremes (one wave: many passes; eight: lanes to spare)
    plans += [tuning.QmvPlan("gemv", 1, n // (c * groups(w)), w) for c in (2, 4) for w in (1, 8)
              if n % (c * groups(w)) == 0]
    if nproj == 1 and chunks <= 512 and n % (8 * groups(8)) == 0:  # eight columns, one pass
        plans += [tuning.QmvPlan("gemv", 1, n // (8 * groups(8)), 8)]
    plans = list(dict.fromkeys(plans))
    worst = 0.0
    for plan in plans:
        outs = {}
        for rows in (1, 2, 3, 4):
            print(f"[{case}] plan {plan} rows {rows}", flush=True)
            one_pass = chunks <= 64 * plan.tiles
            cols = n // plan.strips // groups(plan.tiles)
            if not one_pass and nproj * cols * (4 if rows > 2 else rows) > 8:
                continue  # two passes of this many columns and rows would spill registers
            if cols == 8 and rows > 2:
                continue  # eight columns: one projection of up to two rows
            tuning.install_qmv_plan(rows, k, n, g, bits, nproj, tdt, plan)
            a, b = run(mlx, rows), run(packed, rows)
            torch.cuda.synchronize()
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (plan, rows)
            err = O.tolerance_error(torch_to_act(a, dtype), ref[:rows], dtype)
            assert err <= TOL, (plan, rows, err)
            worst = max(worst, err)
            outs[rows] = a
        most = max(outs, default=0)
        for rows, a in outs.items():
            assert torch.equal(a.view(torch.int16), outs[most][:rows].view(torch.int16)), \
                (plan, rows)
    print(f"[{case}] worst tolerance_error {worst:.2e}", flush=True)
