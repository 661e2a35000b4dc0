"""The step-major repack on the GPU: bit-exact against the oracle's reshape, and every
small-row kernel over repacked codes gives exactly the results it gives over MLX's rows (the
same arithmetic in the same order; only the addresses of the code loads differ). Through the
C ABI: mt_affine_repack, mt_affine_{qmv,swiglu,mlp}_repacked."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import metile_amd as mt
from oracle import affine as O
from tests.helpers import act_to_torch, affine_to_torch, torch_to_act, words_to_torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("bits,n,k", [(4, 96, 256), (8, 40, 512), (4, 8960, 1536),
                                      (4, 1536, 8960), (8, 17408, 512)])
def test_repack_is_the_oracle_reshape(bits, n, k):
    rng = np.random.default_rng(n + k + bits)
    w = rng.integers(0, 2**32, size=(n, k * bits // 32), dtype=np.uint64).astype(np.uint32)
    packed = mt.affine_repack(words_to_torch(w), bits=bits)
    torch.cuda.synchronize()
    assert tuple(packed.shape) == (k // 64, n, 2 * bits)
    got = packed.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, O.repack_step_major(w, bits))


# rows: staged kernel (1..16; two-strip workgroups at N = 8960), register kernel (17..32),
# 32-row chunks plus a remainder (40)
@pytest.mark.parametrize("m", [1, 5, 16, 17, 40])
@pytest.mark.parametrize("bits,g,k,n", [(4, 64, 1536, 8960), (4, 64, 8960, 1536),
                                        (4, 128, 512, 256), (8, 64, 512, 320), (8, 32, 256, 96)])
def test_qmv_repacked_equals_native(m, bits, g, k, n):
    if g == 32 and m > 16:
        m = 16  # groups of 32 run on the staged kernel only, in 16-row chunks
    w = affine_to_torch(O.make_affine_weight(n, k, bits, g, 3, 10), "bf16")
    x = act_to_torch(O.make_activations(m, k, 3), "bf16")
    r = act_to_torch(O.make_activations(m, n, 3, tensor_id=3), "bf16")
    packed = mt.affine_repack(w[0], bits=bits)
    for res in (None, r):
        want = mt.affine_qmv(x, *w, group_size=g, bits=bits, residual=res)
        got = mt.affine_qmv(x, packed, w[1], w[2], group_size=g, bits=bits, residual=res)
        assert _same(got, want), (m, bits, g, k, n, res is None)


@pytest.mark.parametrize("m", [1, 8, 16, 24])
@pytest.mark.parametrize("bits,g,dtype", [(4, 64, "bf16"), (4, 64, "f16"), (8, 32, "bf16"),
                                          (8, 128, "bf16")])
def test_swiglu_repacked_equals_native_and_nax_entry(m, bits, g, dtype):
    if g == 32 and m > 16:
        m = 16
    k, n = 1536, 8960
    gate = affine_to_torch(O.make_affine_weight(n, k, bits, g, 4, 10, dtype), dtype)
    up = affine_to_torch(O.make_affine_weight(n, k, bits, g, 4, 12, dtype), dtype)
    x = act_to_torch(O.make_activations(m, k, 4, dtype=dtype), dtype)
    want = mt.affine_swiglu(x, *gate, *up, group_size=g, bits=bits)
    gp = mt.repack_mlx_affine_weight(*gate, bits=bits)
    upk = mt.repack_mlx_affine_weight(*up, bits=bits)
    got = mt.mlx_affine_swiglu_qmv_nax(x, *gp, *upk, output_features=n, group_size=g, bits=bits)
    assert _same(got, want)
    if m == 1:
        one = mt.mlx_affine_qmv_nax(x, *gp, output_features=n, group_size=g, bits=bits)
        assert _same(one, mt.mlx_affine_qmv(x, *gate, group_size=g, bits=bits))


@pytest.mark.parametrize("m", [1, 3, 16, 33])
def test_mlp_repacked_equals_native(m):
    h, i = 1536, 8960
    gate = affine_to_torch(O.make_affine_weight(i, h, 4, 64, 5, 10), "bf16")
    up = affine_to_torch(O.make_affine_weight(i, h, 4, 64, 5, 12), "bf16")
    down = affine_to_torch(O.make_affine_weight(h, i, 4, 64, 5, 14), "bf16")
    x = act_to_torch(O.make_activations(m, h, 5), "bf16")
    r = act_to_torch(O.make_activations(m, h, 5, tensor_id=3), "bf16")
    want = mt.affine_mlp(x, gate, up, down, residual=r)
    rp = [(mt.affine_repack(t[0]), t[1], t[2]) for t in (gate, up, down)]
    for _ in range(2):  # the second call finds the split-K counters cleared again
        got = mt.affine_mlp(x, *rp, residual=r)
        assert _same(got, want)
    # a layout per stage (mt_affine_mlp_layouts): gate/up in one, down in the other
    assert _same(mt.affine_mlp(x, rp[0], rp[1], down, residual=r), want)
    assert _same(mt.affine_mlp(x, gate, up, rp[2], residual=r), want)


def test_executor_on_repacked_weights_equals_the_native_path():
    # the executors repack once; their results must be those of the MLX-layout kernels
    h, i, m = 1536, 8960, 2
    ts = [affine_to_torch(O.make_affine_weight(i, h, 4, 64, 6, 10), "bf16"),
          affine_to_torch(O.make_affine_weight(i, h, 4, 64, 6, 12), "bf16"),
          affine_to_torch(O.make_affine_weight(h, i, 4, 64, 6, 14), "bf16")]
    x = act_to_torch(O.make_activations(m, h, 6), "bf16")
    r = act_to_torch(O.make_activations(m, h, 6, tensor_id=3), "bf16")
    ex = mt.mlx_affine_mlp_executor(x, *ts[0], *ts[1], *ts[2], r)
    assert _same(ex(x, r), mt.affine_mlp(x, *ts, residual=r))
    ex1 = mt.mlx_affine_mlp_executor(x[:1], *ts[0], *ts[1], *ts[2], r[:1])
    assert _same(ex1(x[:1], r[:1]), mt.affine_mlp(x[:1], *ts, residual=r[:1]))
    sw = mt.mlx_affine_swiglu_executor(x, *ts[0], *ts[1])
    assert _same(sw(x), mt.affine_swiglu(x, *ts[0], *ts[1]))


@pytest.mark.parametrize("m", [1, 3])
def test_mlp_mixed_layouts_with_gemv_plans_f16(m):
    # f16 codes, the down stage on an installed GEMV plan, gate/up on the planner's: every
    # combination of stage layouts gives the bits of the all-MLX call
    from metile_amd import tuning

    h, i = 1024, 3072
    gate = affine_to_torch(O.make_affine_weight(i, h, 4, 64, 8, 10, "f16"), "f16")
    up = affine_to_torch(O.make_affine_weight(i, h, 4, 64, 8, 12, "f16"), "f16")
    down = affine_to_torch(O.make_affine_weight(h, i, 4, 64, 8, 14, "f16"), "f16")
    x = act_to_torch(O.make_activations(m, h, 8, dtype="f16"), "f16")
    r = act_to_torch(O.make_activations(m, h, 8, tensor_id=3, dtype="f16"), "f16")
    tuning.clear_plans()
    try:
        # K = 3072 is 96 chunks: three waves cover two groups of two columns (N / 4 workgroups)
        tuning.install_qmv_plan(m, i, h, 64, 4, 1, torch.float16,
                                tuning.QmvPlan("gemv", 1, h // 4, 3, 1))
        want = mt.affine_mlp(x, gate, up, down, residual=r)
        rp = [(mt.affine_repack(t[0]), t[1], t[2]) for t in (gate, up, down)]
        for g, u, d in ((rp[0], rp[1], down), (gate, up, rp[2]), tuple(rp)):
            assert _same(mt.affine_mlp(x, g, u, d, residual=r), want)
        ref, _ = O.affine_mlp(torch_to_act(x, "f16"), *[
            (t[0].cpu().numpy().view(np.uint32), torch_to_act(t[1], "f16"),
             torch_to_act(t[2], "f16")) for t in (gate, up, down)], 64, 4,
            residual=torch_to_act(r, "f16"), dtype="f16")
        assert O.tolerance_error(torch_to_act(want, "f16"), ref, "f16") <= 2e-3
    finally:
        tuning.clear_plans()
