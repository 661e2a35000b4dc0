"""``BoundMlp``: the executors' per-call fast path over pre-validated weights gives the bits of
``affine_mlp`` over the same weights (it makes the same C-ABI call), and hands inputs it does not
take to ``affine_mlp``, which raises the reference's errors."""

from __future__ import annotations

import pytest
import torch

import metile_amd as mt
from metile_amd.quantized import BoundMlp
from oracle import affine as O
from tests.helpers import act_to_torch, affine_to_torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)


def _weights(h, i, seed):
    return [affine_to_torch(O.make_affine_weight(n, k, 4, 64, seed, t), "bf16")
            for n, k, t in ((i, h, 10), (i, h, 12), (h, i, 14))]


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("layouts", ["mlx/mlx", "repacked/mlx", "repacked/repacked"])
def test_bound_mlp_matches_affine_mlp(layouts):
    h, i = 512, 1024
    g, u, d = _weights(h, i, 3)
    up_l, down_l = layouts.split("/")
    if up_l == "repacked":
        g, u = ((mt.affine_repack(t[0]), t[1], t[2]) for t in (g, u))
    if down_l == "repacked":
        d = (mt.affine_repack(d[0]), d[1], d[2])
    bound = BoundMlp(g, u, d)
    for m in (1, 3, 32, 33):
        x = act_to_torch(O.make_activations(m, h, m), "bf16")
        r = act_to_torch(O.make_activations(m, h, m, tensor_id=3), "bf16")
        assert _same(bound(x, r), mt.affine_mlp(x, g, u, d, residual=r)), m
        assert _same(bound(x), mt.affine_mlp(x, g, u, d)), m
    x3 = act_to_torch(O.make_activations(6, h, 9), "bf16").reshape(2, 3, h)
    assert _same(bound(x3), mt.affine_mlp(x3, g, u, d))
    assert _same(bound(x3[:, ::2]), mt.affine_mlp(x3[:, ::2].contiguous(), g, u, d))


def test_bound_mlp_hands_other_inputs_to_affine_mlp():
    h, i = 256, 512
    bound = BoundMlp(*_weights(h, i, 4))
    with pytest.raises(ValueError, match="incompatible"):
        bound(torch.zeros(2, h + 64, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError, match="residual"):
        bound(torch.zeros(2, h, dtype=torch.bfloat16, device="cuda"),
              torch.zeros(3, h, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):
        bound(torch.zeros(2, h, dtype=torch.float16, device="cuda"))
