"""The weight-format kernels at seeded random shapes and value distributions, on the GPU through
the C ABI, bit for bit against the oracle: the affine quantizer (``mt_affine_quantize``), the
dequantizer (``mt_affine_dequantize``, fp32 ``q * s + b``) and the step-major repack
(``mt_affine_repack``). Shapes: N from 1 to 300 rows, K a multiple of 64 (and of the group) up
to 4096, groups of 32/64/128, 4 and 8 bits, bf16 and f16. Values: normal at scales from 1e-6 to
30, heavy-tailed (Student t, 2 degrees of freedom), groups of one repeated value, integers, and
sparse rows (90% zeros).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import metile_amd as mt
from oracle import affine as O
from tests.helpers import act_to_torch, torch_to_act

pytestmark = pytest.mark.gpu

KINDS = ("normal", "heavy", "constant", "integers", "sparse")


def _cases():
    rng = np.random.RandomState(5150)
    out = []
    for i in range(24):
        g = int(rng.choice([32, 64, 128]))
        k = int(rng.randint(1, 33)) * 128 if g == 128 else int(rng.randint(1, 65)) * 64
        n = int(rng.randint(1, 301))
        bits = int(rng.choice([4, 8]))
        dtype = "f16" if rng.randint(3) == 0 else "bf16"
        kind = KINDS[i % len(KINDS)]
        scale = float(10.0 ** rng.uniform(-6, 1.5))
        out.append((n, k, g, bits, dtype, kind, scale))
    return out


def _values(n, k, g, kind, scale, seed, dtype):
    rng = np.random.default_rng(seed)
    if kind == "normal":
        v = rng.standard_normal((n, k)) * scale
    elif kind == "heavy":
        v = rng.standard_t(2, (n, k)) * scale
    elif kind == "constant":
        v = np.repeat(rng.standard_normal((n, k // g)) * scale, g, axis=1)
    elif kind == "integers":
        v = rng.integers(-20, 21, (n, k)).astype(np.float64)
    else:
        v = rng.standard_normal((n, k)) * scale * (rng.random((n, k)) < 0.1)
    if dtype == "f16":
        v = np.clip(v, -60000.0, 60000.0)
    return O.from_f32(v.astype(np.float32), dtype)


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)


@pytest.mark.parametrize("case", _cases(), ids=lambda c: "x".join(map(str, c[:6])))
def test_quantize_dequantize_repack_bit_exact(case):
    n, k, g, bits, dtype, kind, scale = case
    w = _values(n, k, g, kind, scale, n * 31 + k, dtype)
    w_q, s, b = mt.affine_quantize(act_to_torch(w, dtype), group_size=g, bits=bits)
    ow, os_, ob = O.affine_quantize(w, g, bits, dtype)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(w_q.cpu().numpy().view(np.uint32), ow)
    np.testing.assert_array_equal(torch_to_act(s, dtype), os_)
    np.testing.assert_array_equal(torch_to_act(b, dtype), ob)

    deq = mt.affine_dequantize(w_q, s, b, group_size=g, bits=bits).cpu().numpy()
    want = O.dequantize(ow, os_, ob, g, bits, dtype).astype(np.float32)
    np.testing.assert_array_equal(deq.view(np.uint32), want.view(np.uint32))

    packed = mt.affine_repack(w_q, bits=bits).cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(packed.reshape(-1), O.repack_step_major(ow, bits).reshape(-1))
    print(f"[format {case}] bit-exact", flush=True)
