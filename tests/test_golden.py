"""The committed golden fixtures are reproduced exactly by the oracle (CPU)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import affine as O

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.mark.parametrize("name", sorted(p.stem for p in GOLDEN.glob("qmv_*.npz")))
def test_qmv_fixture_reproduced(name):
    d = np.load(GOLDEN / f"{name}.npz")
    m, k, n, bits, g = (int(v) for v in d["meta"])
    res = d["residual"] if "residual" in d else None
    ref = O.affine_qmv(d["x"], d["w_q"], d["scales"], d["biases"], g, bits, residual=res)
    np.testing.assert_array_equal(ref, d["ref"])
    assert d["x"].shape == (m, k) and d["w_q"].shape == (n, k * bits // 32)


def test_swiglu_and_mlp_fixtures_reproduced():
    d = np.load(GOLDEN / "swiglu_int4_g64_m4_k256_n64.npz")
    ref = O.affine_swiglu(d["x"], (d["gw"], d["gs"], d["gb"]), (d["uw"], d["us"], d["ub"]), 64, 4)
    np.testing.assert_array_equal(ref, d["ref"])
    d = np.load(GOLDEN / "mlp_int4_g64_m2_h128_i192.npz")
    ref, hid = O.affine_mlp(d["x"], (d["gw"], d["gs"], d["gb"]), (d["uw"], d["us"], d["ub"]),
                            (d["dw"], d["ds"], d["db"]), 64, 4, residual=d["residual"])
    np.testing.assert_array_equal(ref, d["ref"])
    np.testing.assert_array_equal(hid, d["hidden"])


def test_kat_fixture_matches_reference_expectation():
    d = np.load(GOLDEN / "kat_seed211_f16.npz")
    got = O.affine_qmv(d["x"], d["w_q"], d["scales"], d["biases"], 64, 4, dtype="f16",
                       acc=np.float32)
    np.testing.assert_array_equal(O.from_f32(got.astype(np.float32), "f16"), d["expected"])
    assert O.tolerance_error(d["expected"], d["ref"], "f16") <= 2e-3
