"""Parity at larger decoder shapes than the BASELINE configs, through the C ABI, with the
planner's plans (tuning is off in the test session): Llama-3-8B's MLP (hidden 4096,
intermediate 14336) and Qwen2.5-7B's projections (hidden 3584, intermediate 18944), 4-bit,
groups of 64.

These shapes take paths the BASELINE shapes do not: hundreds of column strips (448 and 592,
grids of several rounds), long-K down projections over several K splits (224 and 296 steps of
64), and, at 32 rows, two-strip workgroups. The oracle accumulates in fp32 at these sizes (the
contract's reference for full-size configs); the bars are the other GPU tests' bars."""

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


def _report(name, y, ref, min_exact=0.98):
    err = O.tolerance_error(y, ref, "bf16")
    exact = np.mean(O.to_f32(y, "bf16") == O.to_f32(O.from_f32(ref.astype(np.float32), "bf16"),
                                                     "bf16"))
    print(f"[{name}] tolerance_error={err:.3e} exact_fraction={exact:.5f}", flush=True)
    assert err <= TOL, (name, err)
    assert exact >= min_exact, (name, exact)


@functools.lru_cache(maxsize=1)
def _llama_mlp():
    h, i = 4096, 14336
    weights = tuple(O.make_affine_weight(n, k, 4, 64, 21, 10 + 2 * p)
                    for p, (n, k) in enumerate(((i, h), (i, h), (h, i))))
    return h, i, weights, tuple(affine_to_torch(w, "bf16") for w in weights)


@pytest.mark.parametrize("m", [1, 3, 16, 32])
def test_llama3_8b_mlp(m):
    h, i, (gate, up, down), (gt, ut, dt) = _llama_mlp()
    x = O.make_activations(m, h, 21)
    res = O.make_activations(m, h, 21, tensor_id=3)
    xt, rt = act_to_torch(x, "bf16"), act_to_torch(res, "bf16")
    for nproj, k, n in ((2, h, i), (1, i, h)):
        print(f"[llama mlp M={m}] plan nproj={nproj}: "
              f"{tuning.qmv_plan(m, k, n, 64, 4, nproj, torch.bfloat16)}", flush=True)
    y = torch_to_act(mt.affine_mlp(xt, gt, ut, dt, residual=rt), "bf16")
    ref, _ = O.affine_mlp(x, gate, up, down, 64, 4, residual=res, acc=np.float32)
    _report(f"llama mlp M={m}", y, ref, min_exact=0.85)
    # stage by stage, as the BASELINE MLP tests: the hidden activation, then the GPU's own
    # hidden activation through the oracle's down projection
    h_gpu = torch_to_act(mt.affine_swiglu(xt, *gt, *ut), "bf16")
    _report(f"llama mlp M={m} hidden", h_gpu,
            O.affine_swiglu(x, gate, up, 64, 4, acc=np.float32))
    _report(f"llama mlp M={m} down(h_gpu)", y,
            O.affine_qmv(h_gpu, *down, 64, 4, residual=res, acc=np.float32))


@pytest.mark.parametrize("m", [1, 7, 32])
def test_qwen25_7b_projections(m):
    h, i = 3584, 18944
    gate = O.make_affine_weight(i, h, 4, 64, 23, 10)
    up = O.make_affine_weight(i, h, 4, 64, 23, 12)
    x = O.make_activations(m, h, 23)
    got = mt.affine_swiglu(act_to_torch(x, "bf16"), *affine_to_torch(gate, "bf16"),
                           *affine_to_torch(up, "bf16"))
    _report(f"qwen7b swiglu M={m}", torch_to_act(got, "bf16"),
            O.affine_swiglu(x, gate, up, 64, 4, acc=np.float32))
    down = O.make_affine_weight(h, i, 4, 64, 23, 14)
    hid = O.make_activations(m, i, 23, tensor_id=5)
    res = O.make_activations(m, h, 23, tensor_id=3)
    got = mt.affine_qmv(act_to_torch(hid, "bf16"), *affine_to_torch(down, "bf16"),
                        residual=act_to_torch(res, "bf16"))
    _report(f"qwen7b down M={m}", torch_to_act(got, "bf16"),
            O.affine_qmv(hid, *down, 64, 4, residual=res, acc=np.float32))
