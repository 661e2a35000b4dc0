"""The column-block kernel (``MT_QMV_BLOCK``) on the GPU, through the C ABI, against the oracle.

Every case installs block plans for its shape and checks the result against the oracle's
(``tolerance_error`` <= 2e-3 and >= 98% (bf16) / 90% (f16) of outputs equal to the correctly
rounded reference), over MLX codes and over repacked codes (bit-identical), at row counts on both
sides of the 16-row tile (1, 3, 16, 17, 32), 4 and 8 bits, bf16 and f16, groups of 64 and 128,
one and two projections (with and without the residual), K unsplit and split (the partial-sum
protocol), blocks from 1 to 4 tiles of 16 columns, ragged block widths, and one to eight waves.
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
def _case(k, n, g, bits, nproj, residual, dtype, rows):
    weights = [O.make_affine_weight(n, k, bits, g, 21, 10 + 2 * p, dtype) for p in range(nproj)]
    x = O.make_activations(rows, k, 21, dtype=dtype)
    res = O.make_activations(rows, n, 21, tensor_id=3, dtype=dtype) if residual else None
    if nproj == 2:
        ref = O.affine_swiglu(x, weights[0], weights[1], g, bits, dtype=dtype)
    else:
        ref = O.affine_qmv(x, *weights[0], g, bits, residual=res, dtype=dtype)
    return weights, x, res, ref


def _run(rows, k, n, g, bits, nproj, residual, dtype, plans):
    weights, x, res, ref = _case(k, n, g, bits, nproj, residual, dtype, rows)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    xt = act_to_torch(x, dtype)
    rt = None if res is None else act_to_torch(res, dtype)
    mlx = [affine_to_torch(w, dtype) for w in weights]
    packed = [(mt.affine_repack(w, bits=bits), s, b) for (w, s, b) in mlx]

    def run(ts):
        if nproj == 2:
            return mt.affine_swiglu(xt, *ts[0], *ts[1], group_size=g, bits=bits)
        return mt.affine_qmv(xt, *ts[0], group_size=g, bits=bits, residual=rt)

    min_exact = 0.98 if dtype == "bf16" else 0.90
    for plan in plans:
        print(f"[{rows}x{k}x{n} g{g} b{bits} p{nproj} {dtype}] plan {plan}", flush=True)
        tuning.install_qmv_plan(rows, k, n, g, bits, nproj, tdt, plan)
        assert tuning.qmv_plan(rows, k, n, g, bits, nproj, tdt) == plan
        a, b = run(mlx), run(packed)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), plan
        y = torch_to_act(a, dtype)
        err = O.tolerance_error(y, ref, dtype)
        exact = np.mean(O.to_f32(y, dtype) == O.to_f32(O.from_f32(ref.astype(np.float32), dtype),
                                                       dtype))
        assert err <= TOL and exact >= min_exact, (plan, err, exact)


def block(ksplit, strips, waves):
    return tuning.QmvPlan("block", ksplit, strips, waves, 0)


@pytest.mark.parametrize("rows", [1, 3, 16, 17, 32])
def test_block_swiglu_4bit_rows(rows):
    # 1536 -> 448: blocks of 28 columns (two tiles, one ragged), of 14 (one tile), and of 56
    # (four tiles; above 16 rows, when two row tiles and two projections leave no room for
    # four, of 37 to 40: three)
    wide = block(1, 8, 4) if rows <= 16 else block(1, 12, 4)
    _run(rows, 1536, 448, 64, 4, 2, False, "bf16",
         [block(1, 16, 8), block(1, 32, 8), wide, block(2, 16, 8)])


@pytest.mark.parametrize("rows", [1, 5, 16, 32])
def test_block_residual_qmv_long_k(rows):
    # 4480 -> 128: 70 K steps over 8 waves, unsplit and over two, five and seven splits (the
    # activations of a split sit in LDS, so more rows need shorter splits)
    plans = {1: [block(1, 8, 8), block(2, 8, 8), block(5, 4, 8), block(1, 2, 4), block(1, 3, 7)],
             5: [block(1, 8, 8), block(2, 8, 8), block(5, 4, 8), block(1, 2, 4), block(1, 3, 7)],
             16: [block(2, 8, 8), block(5, 4, 8), block(2, 3, 7)],
             32: [block(5, 4, 8), block(5, 8, 4), block(7, 3, 7)]}[rows]
    _run(rows, 4480, 128, 64, 4, 1, True, "bf16", plans)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("bits", [4, 8])
def test_block_bits_and_dtypes(bits, dtype):
    _run(8, 1024, 256, 64, bits, 1, False, dtype, [block(1, 8, 8), block(2, 5, 4)])
    _run(8, 1024, 256, 64, bits, 2, False, dtype, [block(1, 8, 8), block(1, 16, 2)])


def test_block_group_128():
    _run(4, 2048, 192, 128, 4, 2, False, "bf16", [block(1, 4, 8), block(2, 6, 8)])
    _run(20, 2048, 192, 128, 8, 1, True, "bf16", [block(1, 4, 8), block(4, 3, 4)])


def test_block_rows_independent_of_batch():
    """A row's output under a block plan does not depend on the other rows of its dispatch."""
    k, n, g, bits = 1536, 256, 64, 4
    weights, x, _, _ = _case(k, n, g, bits, 2, False, "bf16", 32)
    xt = act_to_torch(x, "bf16")
    ws = [affine_to_torch(w, "bf16") for w in weights]
    for bucket in (1, 2, 4, 8, 16, 32):
        tuning.install_qmv_plan(bucket, k, n, g, bits, 2, torch.bfloat16, block(1, 8, 8))
    full = mt.affine_swiglu(xt, *ws[0], *ws[1], group_size=g, bits=bits)
    for r in (0, 7, 15):
        one = mt.affine_swiglu(xt[r:r + 1], *ws[0], *ws[1], group_size=g, bits=bits)
        assert torch.equal(one.view(torch.int16), full[r:r + 1].view(torch.int16)), r


def test_block_plans_listed_and_rejected():
    cands = tuning.qmv_plan_candidates(16, 1536, 8960, 64, 4, 2)
    assert any(p.kernel == "block" for p in cands)
    with pytest.raises(ValueError):  # groups of 32
        tuning.install_qmv_plan(8, 1024, 256, 32, 4, 1, torch.bfloat16, block(1, 8, 8))
    with pytest.raises(ValueError):  # blocks of 128 columns
        tuning.install_qmv_plan(8, 1024, 256, 64, 4, 1, torch.bfloat16, block(1, 2, 8))
    with pytest.raises(ValueError):  # four tiles of two projections over two row tiles
        tuning.install_qmv_plan(32, 1024, 256, 64, 4, 2, torch.bfloat16, block(1, 4, 8))
