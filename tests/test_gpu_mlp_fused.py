"""The one-launch quantized MLP (gate/up and down workgroups of one grid) on the GPU; an
opt-in path (``METILE_AMD_MLP_PATH=fused``), selected explicitly here.

Checks, through the C ABI: parity with the oracle at config 1 and at other shapes, dtypes and
bit widths; agreement with the two-launch composition; that repeated calls, calls interleaved
with other kernels that share the workspace counters, and replays of a captured graph all give
bit-identical results (the hand-off counters return to zero after every call).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import metile_amd as mt
from oracle import affine as O
from tests.helpers import act_to_torch, affine_to_torch, torch_to_act
from tests.test_gpu_affine import _report

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)


def _mlp(x, gate, up, down, g, bits, res, path="fused"):
    old = os.environ.get("METILE_AMD_MLP_PATH")
    os.environ["METILE_AMD_MLP_PATH"] = path
    try:
        y = mt.affine_mlp(x, gate, up, down, group_size=g, bits=bits, residual=res)
        torch.cuda.synchronize()
        return y
    finally:
        if old is None:
            os.environ.pop("METILE_AMD_MLP_PATH")
        else:
            os.environ["METILE_AMD_MLP_PATH"] = old


def _case(m, h, i, bits, g, dtype, cid):
    gate = O.make_affine_weight(i, h, bits, g, cid, 10, dtype)
    up = O.make_affine_weight(i, h, bits, g, cid, 12, dtype)
    down = O.make_affine_weight(h, i, bits, g, cid, 14, dtype)
    x = O.make_activations(m, h, cid, dtype=dtype)
    res = O.make_activations(m, h, cid, tensor_id=3, dtype=dtype)
    return gate, up, down, x, res


@pytest.mark.parametrize("m,h,i,bits,g,dtype", [
    (1, 1536, 8960, 4, 64, "bf16"),    # config 1 shape
    (3, 1536, 8960, 4, 64, "bf16"),
    (16, 1536, 8960, 4, 64, "bf16"),
    (5, 256, 384, 4, 128, "f16"),
    (8, 512, 1024, 8, 64, "bf16"),
    (2, 320, 640, 8, 64, "f16"),
])
def test_fused_mlp_matches_oracle_and_two_launch_path(m, h, i, bits, g, dtype):
    gate, up, down, x, res = _case(m, h, i, bits, g, dtype, cid=m + h)
    ref, _ = O.affine_mlp(x, gate, up, down, g, bits, residual=res, dtype=dtype)
    xt, rt = act_to_torch(x, dtype), act_to_torch(res, dtype)
    gt, ut, dt = (affine_to_torch(t, dtype) for t in (gate, up, down))
    fused = _mlp(xt, gt, ut, dt, g, bits, rt)
    split = _mlp(xt, gt, ut, dt, g, bits, rt, path="split")
    name = f"fused mlp M={m} H={h} I={i} int{bits} g{g} {dtype}"
    _report(name, torch_to_act(fused, dtype), ref, dtype=dtype, min_exact=0.85 if dtype == "bf16" else 0.8)
    # Same hidden activation; only the down projection's K split boundaries may differ.
    _report(name + " vs two-launch", torch_to_act(fused, dtype),
            O.to_f32(torch_to_act(split, dtype), dtype).astype(np.float64), dtype=dtype,
            min_exact=0.97)


def test_fused_mlp_repeats_interleaved_and_graph_replays():
    m, h, i = 2, 1536, 8960
    gate, up, down, x, res = _case(m, h, i, 4, 64, "bf16", cid=1)
    xt, rt = act_to_torch(x, "bf16"), act_to_torch(res, "bf16")
    gt, ut, dt = (affine_to_torch(t, "bf16") for t in (gate, up, down))
    first = _mlp(xt, gt, ut, dt, 64, 4, rt)
    for _ in range(3):
        # Other kernels that use the workspace counter region between fused calls.
        mt.affine_qmv(xt, *gt, group_size=64, bits=4)
        mt.affine_qmv(torch.randn(m, i, device="cuda").to(torch.bfloat16), *dt, group_size=64,
                      bits=4)
        again = _mlp(xt, gt, ut, dt, 64, 4, rt)
        assert torch.equal(again.view(torch.int16), first.view(torch.int16))

    stream = torch.cuda.Stream()
    out = [None]
    os.environ["METILE_AMD_MLP_PATH"] = "fused"
    try:
        with torch.cuda.stream(stream):
            out[0] = mt.affine_mlp(xt, gt, ut, dt, residual=rt)  # workspace for this stream
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                out[0] = mt.affine_mlp(xt, gt, ut, dt, residual=rt)
    finally:
        os.environ.pop("METILE_AMD_MLP_PATH")
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0].view(torch.int16), first.view(torch.int16))
        eager = _mlp(xt, gt, ut, dt, 64, 4, rt)
        assert torch.equal(eager.view(torch.int16), first.view(torch.int16))
