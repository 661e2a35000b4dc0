"""Writes the small golden fixtures under tests/golden/ from the NumPy oracle.

Run from the repo root: ``python tests/golden/make_golden.py``. Each ``.npz`` holds the inputs
(bf16/f16 as raw bits), the unrounded float64 reference and the reference rounded to the
activation dtype. ``kat_seed211_f16.npz`` restates the reference's own known-answer test
(tests/test_affine_quantized.py:120-163: seed 211, 64x64, f16, one group per row).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import affine as O  # noqa: E402


def affine_case(name, m, k, n, bits, g, config_id, residual=False):
    w_q, s, b = O.make_affine_weight(n, k, bits, g, config_id, 10)
    x = O.make_activations(m, k, config_id)
    res = O.make_activations(m, n, config_id, tensor_id=3) if residual else None
    ref = O.affine_qmv(x, w_q, s, b, g, bits, residual=res)
    arrays = dict(x=x, w_q=w_q, scales=s, biases=b, ref=ref,
                  expected=O.from_f32(ref.astype(np.float32), "bf16"),
                  meta=np.array([m, k, n, bits, g]))
    if residual:
        arrays["residual"] = res
    np.savez_compressed(HERE / f"{name}.npz", **arrays)


def swiglu_case(name, m, k, n, bits, g, config_id):
    gate = O.make_affine_weight(n, k, bits, g, config_id, 10)
    up = O.make_affine_weight(n, k, bits, g, config_id, 12)
    x = O.make_activations(m, k, config_id)
    ref = O.affine_swiglu(x, gate, up, g, bits)
    np.savez_compressed(HERE / f"{name}.npz", x=x, gw=gate[0], gs=gate[1], gb=gate[2], uw=up[0],
                        us=up[1], ub=up[2], ref=ref,
                        expected=O.from_f32(ref.astype(np.float32), "bf16"),
                        meta=np.array([m, k, n, bits, g]))


def mlp_case(name, m, h, i, bits, g, config_id):
    gate = O.make_affine_weight(i, h, bits, g, config_id, 10)
    up = O.make_affine_weight(i, h, bits, g, config_id, 12)
    down = O.make_affine_weight(h, i, bits, g, config_id, 14)
    x = O.make_activations(m, h, config_id)
    res = O.make_activations(m, h, config_id, tensor_id=3)
    ref, hid = O.affine_mlp(x, gate, up, down, g, bits, residual=res)
    np.savez_compressed(HERE / f"{name}.npz", x=x, residual=res, gw=gate[0], gs=gate[1],
                        gb=gate[2], uw=up[0], us=up[1], ub=up[2], dw=down[0], ds=down[1],
                        db=down[2], hidden=hid, ref=ref,
                        expected=O.from_f32(ref.astype(np.float32), "bf16"),
                        meta=np.array([m, h, i, bits, g]))


def kat_seed211():
    k = n = 64
    random = np.random.default_rng(211)
    activations = random.normal(size=(1, k)).astype(np.float16)
    quantized = random.integers(0, 16, size=(n, k), dtype=np.uint8)
    scales = random.uniform(0.01, 0.2, size=(1, n)).astype(np.float16)
    biases = random.uniform(-0.5, 0.5, size=(1, n)).astype(np.float16)
    expected_weight = (quantized.astype(np.float32) * scales.T.astype(np.float32)
                       + biases.T.astype(np.float32))
    expected = (activations.astype(np.float32) @ expected_weight.T).astype(np.float16)
    ref = activations.astype(np.float64) @ expected_weight.astype(np.float64).T
    np.savez_compressed(HERE / "kat_seed211_f16.npz", x=activations,
                        w_q=O.pack_codes(quantized, 4), scales=scales.T.copy(),
                        biases=biases.T.copy(), expected=expected, ref=ref,
                        dequantized=expected_weight)


def main():
    affine_case("qmv_int4_g64_m3_k256_n64", 3, 256, 64, 4, 64, 100)
    affine_case("qmv_int4_g64_m1_k1536_n96_residual", 1, 1536, 96, 4, 64, 101, residual=True)
    affine_case("qmv_int8_g128_m5_k512_n96", 5, 512, 96, 8, 128, 102)
    affine_case("qmv_int8_g64_m17_k256_n32", 17, 256, 32, 8, 64, 103)
    swiglu_case("swiglu_int4_g64_m4_k256_n64", 4, 256, 64, 4, 64, 104)
    mlp_case("mlp_int4_g64_m2_h128_i192", 2, 128, 192, 4, 64, 105)
    kat_seed211()


if __name__ == "__main__":
    main()
