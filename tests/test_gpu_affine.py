"""Parity of the gfx950 affine kernels (through the C ABI) with the NumPy oracle.

Contract: dequantization is bit-exact; projection outputs are within 2e-3 (max-abs normalised,
after the unavoidable final rounding to the activation dtype; ``oracle.affine.tolerance_error``)
of an fp64 / fp32-accumulated reference over the identical dequantized weights. The tests also
require that almost every output equals the correctly rounded reference, which is far tighter.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import metile_amd as mt
from oracle import affine as O
from tests.helpers import act_to_torch, affine_to_torch, torch_to_act, words_to_torch

pytestmark = pytest.mark.gpu

TOL = 2e-3
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)


def _report(name, y, ref, dtype="bf16", min_exact=None):
    err = O.tolerance_error(y, ref, dtype)
    exact = np.mean(O.to_f32(y, dtype) == O.to_f32(O.from_f32(ref.astype(np.float32), dtype),
                                                   dtype))
    print(f"[{name}] tolerance_error={err:.3e} plain={O.plain_error(y, ref, dtype):.3e} "
          f"exact_fraction={exact:.5f}", flush=True)
    assert err <= TOL, (name, err)
    # f16 keeps 3 more mantissa bits than bf16, so fp32 accumulation noise flips more of its
    # roundings; the contract above is the tolerance, this is a far stricter sanity bar.
    if min_exact is None:
        min_exact = 0.98 if dtype == "bf16" else 0.90
    assert exact >= min_exact, (name, exact)


def _qmv_case(m, k, n, bits, g, dtype="bf16", config_id=0, residual=False, acc=np.float64):
    w = O.make_affine_weight(n, k, bits, g, config_id, 10, dtype)
    x = O.make_activations(m, k, config_id, dtype=dtype)
    res = O.make_activations(m, n, config_id, tensor_id=3, dtype=dtype) if residual else None
    ref = O.affine_qmv(x, *w, g, bits, residual=res, dtype=dtype, acc=acc)
    wt = affine_to_torch(w, dtype)
    rt = None if res is None else act_to_torch(res, dtype)
    y = mt.affine_qmv(act_to_torch(x, dtype), *wt, group_size=g, bits=bits, residual=rt)
    torch.cuda.synchronize()
    return torch_to_act(y, dtype), ref


# ---- dequantization ------------------------------------------------------------------------


@pytest.mark.parametrize("bits,g", [(4, 64), (4, 32), (8, 128), (8, 64)])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_dequantize_is_bit_exact(bits, g, dtype):
    n, k = 96, 512
    w_q, s, b = O.make_affine_weight(n, k, bits, g, 9, 10, dtype)
    # general affine parameters, not only the b = -zero*s recipe
    b = O.from_f32(O.rng(9, 20).uniform(-1, 1, size=s.shape).astype(np.float32), dtype)
    got = mt.affine_dequantize(*affine_to_torch((w_q, s, b), dtype), group_size=g, bits=bits)
    want = O.dequantize(w_q, s, b, g, bits, dtype)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


# ---- single projection ---------------------------------------------------------------------


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 16, 17, 31, 32])
def test_qmv_int4_config0_rows(m):
    y, ref = _qmv_case(m, 1536, 8960, 4, 64, config_id=0)
    _report(f"qmv int4 M={m} K=1536 N=8960", y, ref)


@pytest.mark.parametrize("m,k,n,bits,g", [
    (1, 64, 32, 4, 64),      # smallest shape: one step, one strip
    (3, 256, 64, 4, 64),
    (2, 256, 64, 8, 64),
    (7, 512, 96, 8, 128),
    (4, 1024, 160, 4, 128),
    (12, 4096, 64, 4, 64),   # long K, few strips -> split-K
    (33, 512, 64, 4, 64),    # more than one 32-row chunk
    (70, 256, 96, 8, 64),
])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_qmv_shapes_and_dtypes(m, k, n, bits, g, dtype):
    y, ref = _qmv_case(m, k, n, bits, g, dtype=dtype, config_id=m + k)
    _report(f"qmv {dtype} int{bits} g{g} M={m} K={k} N={n}", y, ref, dtype)


# Groups of 32: two groups per 64-wide K step (two MFMA chains per step), 16-row chunks, and
# for long K more K splits (at most 31 steps per split).
@pytest.mark.parametrize("m,k,n,bits,dtype", [
    (1, 1024, 160, 4, "bf16"),
    (5, 1024, 96, 8, "bf16"),
    (16, 2048, 64, 8, "f16"),
    (21, 512, 128, 4, "bf16"),    # a 16-row chunk and a 5-row chunk
    (3, 5120, 256, 8, "bf16"),    # 80 steps -> at least three K splits
])
def test_qmv_group32(m, k, n, bits, dtype):
    y, ref = _qmv_case(m, k, n, bits, 32, dtype=dtype, config_id=m + k + n)
    _report(f"qmv {dtype} int{bits} g32 M={m} K={k} N={n}", y, ref, dtype)


def test_mlp_int8_group32():
    gate = O.make_affine_weight(384, 256, 8, 32, 6, 10)
    up = O.make_affine_weight(384, 256, 8, 32, 6, 12)
    down = O.make_affine_weight(256, 384, 8, 32, 6, 14)
    x = O.make_activations(4, 256, 6)
    res = O.make_activations(4, 256, 6, tensor_id=3)
    ref, _ = O.affine_mlp(x, gate, up, down, 32, 8, residual=res)
    y = mt.affine_mlp(act_to_torch(x, "bf16"), affine_to_torch(gate, "bf16"),
                      affine_to_torch(up, "bf16"), affine_to_torch(down, "bf16"),
                      group_size=32, bits=8, residual=act_to_torch(res, "bf16"))
    _report("mlp int8 g32 M=4", torch_to_act(y, "bf16"), ref, min_exact=0.85)


@pytest.mark.parametrize("m", [1, 5, 32])
def test_residual_qmv_config1_down(m):
    y, ref = _qmv_case(m, 8960, 1536, 4, 64, config_id=1, residual=True)
    _report(f"residual qmv M={m} K=8960 N=1536", y, ref)


@pytest.mark.parametrize("m", [1, 8, 16])
def test_qmv_int8_config3(m):
    y, ref = _qmv_case(m, 5120, 17408, 8, 64, config_id=3, acc=np.float32)
    _report(f"qmv int8 M={m} K=5120 N=17408", y, ref)


def test_mlx_residual_entry_point_and_leading_dims():
    k, n = 512, 64
    w = O.make_affine_weight(n, k, 4, 64, 5, 10)
    x = O.make_activations(6, k, 5)
    res = O.make_activations(6, n, 5, tensor_id=3)
    ref = O.affine_qmv(x, *w, 64, 4, residual=res)
    xt = act_to_torch(x, "bf16").reshape(2, 3, k)
    rt = act_to_torch(res, "bf16").reshape(2, 3, n)
    y = mt.mlx_affine_residual_qmv(xt, *affine_to_torch(w, "bf16"), rt)
    assert tuple(y.shape) == (2, 3, n)
    _report("mlx_affine_residual_qmv [2,3,K]", torch_to_act(y.reshape(6, n), "bf16"), ref)


def test_empty_rows_return_empty():
    w = affine_to_torch(O.make_affine_weight(64, 256, 4, 64, 0, 10), "bf16")
    x = torch.zeros(0, 256, dtype=torch.bfloat16, device="cuda")
    assert tuple(mt.affine_qmv(x, *w).shape) == (0, 64)


def test_results_are_deterministic():
    w = affine_to_torch(O.make_affine_weight(1536, 8960, 4, 64, 1, 14), "bf16")
    x = act_to_torch(O.make_activations(4, 8960, 1), "bf16")
    a = mt.affine_qmv(x, *w)
    b = mt.affine_qmv(x, *w)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_reference_kat_seed211_f16():
    d = np.load(GOLDEN / "kat_seed211_f16.npz")
    y = mt.affine_qmv(act_to_torch(d["x"], "f16"), words_to_torch(d["w_q"]),
                      act_to_torch(d["scales"], "f16"), act_to_torch(d["biases"], "f16"))
    got = torch_to_act(y, "f16")
    # the reference test's own bar (rtol = atol = 3e-2) and the build's contract
    np.testing.assert_allclose(got.astype(np.float32), d["expected"].astype(np.float32),
                               rtol=3e-2, atol=3e-2)
    _report("KAT seed 211 f16", got, d["ref"], "f16")


# ---- SwiGLU and MLP ------------------------------------------------------------------------


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16, 32])
def test_swiglu_config1(m):
    gate = O.make_affine_weight(8960, 1536, 4, 64, 1, 10)
    up = O.make_affine_weight(8960, 1536, 4, 64, 1, 12)
    x = O.make_activations(m, 1536, 1)
    ref = O.affine_swiglu(x, gate, up, 64, 4)
    h = mt.mlx_affine_swiglu(act_to_torch(x, "bf16"), *affine_to_torch(gate, "bf16"),
                             *affine_to_torch(up, "bf16"))
    _report(f"swiglu M={m}", torch_to_act(h, "bf16"), ref)


@pytest.mark.parametrize("bits,g", [(8, 64), (8, 128), (8, 32)])
def test_swiglu_int8(bits, g):
    gate = O.make_affine_weight(512, 1024, bits, g, 4, 10)
    up = O.make_affine_weight(512, 1024, bits, g, 4, 12)
    x = O.make_activations(3, 1024, 4)
    ref = O.affine_swiglu(x, gate, up, g, bits)
    h = mt.mlx_affine_swiglu(act_to_torch(x, "bf16"), *affine_to_torch(gate, "bf16"),
                             *affine_to_torch(up, "bf16"), bits=bits, group_size=g)
    _report(f"swiglu int{bits} g{g}", torch_to_act(h, "bf16"), ref)


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16, 32])
def test_mlp_executor_config1(m):
    gate = O.make_affine_weight(8960, 1536, 4, 64, 1, 10)
    up = O.make_affine_weight(8960, 1536, 4, 64, 1, 12)
    down = O.make_affine_weight(1536, 8960, 4, 64, 1, 14)
    x = O.make_activations(m, 1536, 1)
    res = O.make_activations(m, 1536, 1, tensor_id=3)
    ref, hid = O.affine_mlp(x, gate, up, down, 64, 4, residual=res)
    xt, rt = act_to_torch(x, "bf16"), act_to_torch(res, "bf16")
    gt, ut, dt = (affine_to_torch(t, "bf16") for t in (gate, up, down))
    ex = mt.mlx_affine_mlp_executor(xt, *gt, *ut, *dt, rt)
    y = torch_to_act(ex(xt, rt), "bf16")
    # End to end: the contract. The hidden activation is rounded to bf16 between the two
    # kernels, so a one-ulp difference in h legitimately moves some output roundings.
    _report(f"mlp M={m}", y, ref, min_exact=0.85)
    # Stage by stage: the GPU's own hidden activation through the oracle's down projection
    # must reproduce the executor's output as tightly as a single projection.
    h_gpu = torch_to_act(mt.affine_swiglu(xt, *gt, *ut), "bf16")
    _report(f"mlp M={m} hidden", h_gpu, O.affine_swiglu(x, gate, up, 64, 4))
    _report(f"mlp M={m} down(h_gpu)", y, O.affine_qmv(h_gpu, *down, 64, 4, residual=res))


# ---- golden fixtures -----------------------------------------------------------------------


@pytest.mark.parametrize("name", sorted(p.stem for p in GOLDEN.glob("qmv_*.npz")))
def test_golden_qmv(name):
    d = np.load(GOLDEN / f"{name}.npz")
    m, k, n, bits, g = (int(v) for v in d["meta"])
    res = act_to_torch(d["residual"], "bf16") if "residual" in d else None
    y = mt.affine_qmv(act_to_torch(d["x"], "bf16"), words_to_torch(d["w_q"]),
                      act_to_torch(d["scales"], "bf16"), act_to_torch(d["biases"], "bf16"),
                      group_size=g, bits=bits, residual=res)
    _report(name, torch_to_act(y, "bf16"), d["ref"])


def test_golden_swiglu_and_mlp():
    d = np.load(GOLDEN / "swiglu_int4_g64_m4_k256_n64.npz")
    h = mt.affine_swiglu(act_to_torch(d["x"], "bf16"),
                         *affine_to_torch((d["gw"], d["gs"], d["gb"]), "bf16"),
                         *affine_to_torch((d["uw"], d["us"], d["ub"]), "bf16"))
    _report("golden swiglu", torch_to_act(h, "bf16"), d["ref"])
    d = np.load(GOLDEN / "mlp_int4_g64_m2_h128_i192.npz")
    y = mt.affine_mlp(act_to_torch(d["x"], "bf16"),
                      affine_to_torch((d["gw"], d["gs"], d["gb"]), "bf16"),
                      affine_to_torch((d["uw"], d["us"], d["ub"]), "bf16"),
                      affine_to_torch((d["dw"], d["ds"], d["db"]), "bf16"),
                      residual=act_to_torch(d["residual"], "bf16"))
    _report("golden mlp", torch_to_act(y, "bf16"), d["ref"], min_exact=0.85)


def test_workspace_is_never_created_inside_graph_capture():
    """A split-K call (the down projection at 8 rows: 5 K splits) on a stream without a
    workspace raises under capture instead of recording the workspace's zero fill into the
    graph; after one call outside capture, graphs captured on that stream replay correctly in
    any order, with eager calls between replays."""
    k, n, m = 8960, 1536, 8
    w = affine_to_torch(O.make_affine_weight(n, k, 4, 64, 9, 10), "bf16")
    x = act_to_torch(O.make_activations(m, k, 9), "bf16")
    x2 = act_to_torch(O.make_activations(m, k, 9, tensor_id=4), "bf16")
    want1 = mt.affine_qmv(x, *w)
    want2 = mt.affine_qmv(x2, *w)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    g0 = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="outside graph capture"):
        with torch.cuda.graph(g0, stream=stream):
            mt.affine_qmv(x, *w)
    with torch.cuda.stream(stream):
        mt.affine_qmv(x, *w)  # creates the stream's workspace, outside capture
    stream.synchronize()
    outs = {}
    graphs = []
    for key, xin in (("a", x), ("b", x2)):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            outs[key] = mt.affine_qmv(xin, *w)
        graphs.append(g)
    for _ in range(3):
        graphs[1].replay()
        graphs[0].replay()
        torch.cuda.synchronize()
        assert torch.equal(outs["b"].view(torch.int16), want2.view(torch.int16))
        assert torch.equal(outs["a"].view(torch.int16), want1.view(torch.int16))
        with torch.cuda.stream(stream):
            mid = mt.affine_qmv(x2, *w)
        stream.synchronize()
        assert torch.equal(mid.view(torch.int16), want2.view(torch.int16))
