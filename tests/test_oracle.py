"""Pins the NumPy oracle (CPU only) against known answers, closed forms, brute force and an
independent implementation (torch CPU), so that a plausible mistake in it fails a test."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import affine as O


# ---- bf16 rounding ------------------------------------------------------------------------


def _torch_bf16_bits(f32: np.ndarray) -> np.ndarray:
    return torch.from_numpy(f32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_bf16_rounding_matches_torch_on_edge_patterns():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    # ties (low half exactly 0x8000) with both mantissa parities, denormals, infinities
    ties = (rng.integers(0, 2**16, size=4096, dtype=np.uint32) << 16) | np.uint32(0x8000)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x00000001, 0x007FFFFF,
                        0x3F808000, 0x3F818000, 0x7F7FFFFF, 0x477FE000], dtype=np.uint32)
    f = np.concatenate([bits, ties, special]).view(np.float32)
    f = f[~np.isnan(f)]
    np.testing.assert_array_equal(O.f32_to_bf16_bits(f), _torch_bf16_bits(f))


def test_bf16_widening_is_exact():
    b = np.arange(0, 2**16, dtype=np.uint32).astype(np.uint16)
    f = O.bf16_bits_to_f32(b)
    ok = ~np.isnan(f)
    np.testing.assert_array_equal(O.f32_to_bf16_bits(f[ok]), b[ok])


def test_half_ulp_bf16_known_values():
    np.testing.assert_allclose(O.half_ulp(np.array([1.0, 1.5, 2.0, 255.0, 0.75])),
                               [2**-8, 2**-8, 2**-7, 2**-1, 2**-9])


# ---- packing ------------------------------------------------------------------------------


def test_unpack_hand_built_words():
    w = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    np.testing.assert_array_equal(O.unpack_codes(w, 4)[0], np.arange(16))
    w8 = np.array([[0x03020100, 0xFFFE8180]], dtype=np.uint32)
    np.testing.assert_array_equal(O.unpack_codes(w8, 8)[0], [0, 1, 2, 3, 0x80, 0x81, 0xFE, 0xFF])


def test_pack_hand_built_codes():
    codes = np.arange(16, dtype=np.uint32)[None, :]
    np.testing.assert_array_equal(O.pack_codes(codes, 4), [[0x76543210, 0xFEDCBA98]])


@settings(max_examples=60, deadline=None)
@given(bits=st.sampled_from([4, 8]), n=st.integers(1, 5), words=st.integers(1, 6),
       seed=st.integers(0, 2**31))
def test_pack_unpack_round_trip(bits, n, words, seed):
    per = 32 // bits
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 1 << bits, size=(n, words * per), dtype=np.uint32)
    packed = O.pack_codes(codes, bits)
    assert packed.shape == (n, words)
    np.testing.assert_array_equal(O.unpack_codes(packed, bits), codes)
    raw = rng.integers(0, 2**32, size=(n, words), dtype=np.uint64).astype(np.uint32)
    np.testing.assert_array_equal(O.pack_codes(O.unpack_codes(raw, bits), bits), raw)


# ---- step-major repack --------------------------------------------------------------------


@pytest.mark.parametrize("bits", [4, 8])
def test_repack_puts_each_rows_64_codes_at_their_step(bits):
    # row n holds code (n + k // 64) % 2^bits at k: the chunk [t, n] must unpack to n + t only
    n, k = 5, 256
    codes = (np.arange(n)[:, None] + (np.arange(k) // 64)[None, :]) % (1 << bits)
    packed = O.repack_step_major(O.pack_codes(codes, bits), bits)
    assert packed.shape == (k // 64, n, 2 * bits)
    for t in range(k // 64):
        chunk_codes = O.unpack_codes(packed[t], bits)  # [n, 64]
        np.testing.assert_array_equal(chunk_codes, np.broadcast_to(
            ((np.arange(n) + t) % (1 << bits))[:, None], (n, 64)))


@pytest.mark.parametrize("bits", [4, 8])
def test_repack_matches_a_brute_force_index_loop_and_inverts(bits):
    rng = np.random.default_rng(17)
    n, k = 7, 192
    w = rng.integers(0, 2**32, size=(n, k * bits // 32), dtype=np.uint64).astype(np.uint32)
    packed = O.repack_step_major(w, bits)
    chunk = 2 * bits
    for t in range(k // 64):
        for row in range(n):
            for e in range(chunk):
                assert packed[t, row, e] == w[row, t * chunk + e]
    np.testing.assert_array_equal(packed.transpose(1, 0, 2).reshape(n, -1), w)


# ---- dequantization -----------------------------------------------------------------------


@pytest.mark.parametrize("bits,zero", [(4, 8.0), (8, 128.0)])
def test_dequantize_closed_form_baseline_recipe(bits, zero):
    w_q, s, b = O.make_affine_weight(48, 256, bits, 64, config_id=7, tensor_id=3)
    got = O.dequantize(w_q, s, b, 64, bits)
    q = O.unpack_codes(w_q, bits).astype(np.float64)
    s64 = np.repeat(O.bf16_bits_to_f32(s).astype(np.float64), 64, axis=1)
    expected = (q - zero) * s64  # exact: (q - zero) has <= 8 bits, s has 8
    np.testing.assert_array_equal(got.astype(np.float64), expected)


def _brute_force_qmv(x, w_q, s, b, k, group_size, bits):
    """Literal loop of kernels/affine_qmv.py:32-53 (per word, per element), float64."""
    per = 32 // bits
    words_per_row = k // per
    words_per_group = group_size // per
    n = w_q.shape[0]
    out = np.zeros((x.shape[0], n))
    for row in range(x.shape[0]):
        for col in range(n):
            acc = 0.0
            for wi in range(words_per_row):
                packed = int(w_q[col, wi])
                g = wi // words_per_group
                scale = float(s[col, g])
                bias = float(b[col, g])
                for e in range(per):
                    q = (packed >> (e * bits)) & ((1 << bits) - 1)
                    acc += float(x[row, wi * per + e]) * (q * scale + bias)
            out[row, col] = acc
    return out


@pytest.mark.parametrize("bits,group_size", [(4, 64), (8, 64), (4, 128), (8, 32)])
def test_qmv_matches_brute_force_loop(bits, group_size):
    k, n, m = 256, 6, 3
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 1 << bits, size=(n, k), dtype=np.uint32)
    w_q = O.pack_codes(codes, bits)
    s = O.f32_to_bf16_bits(rng.uniform(0.01, 0.1, size=(n, k // group_size)).astype(np.float32))
    b = O.f32_to_bf16_bits(rng.uniform(-0.5, 0.5, size=(n, k // group_size)).astype(np.float32))
    x = O.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    got = O.affine_qmv(x, w_q, s, b, group_size, bits)
    ref = _brute_force_qmv(O.bf16_bits_to_f32(x), w_q, O.bf16_bits_to_f32(s),
                           O.bf16_bits_to_f32(b), k, group_size, bits)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_reference_known_answer_seed_211():
    """Restates tests/test_affine_quantized.py:120-163: seed 211, 64x64, f16, one group per
    output row; the reference packs K-major nibble pairs, this oracle takes MLX output-major
    words, so the codes are repacked and the reference's own fp32 expectation is compared."""
    k = n = 64
    random = np.random.default_rng(211)
    activations = random.normal(size=(1, k)).astype(np.float16)
    quantized = random.integers(0, 16, size=(n, k), dtype=np.uint8)
    scales = random.uniform(0.01, 0.2, size=(1, n)).astype(np.float16)
    biases = random.uniform(-0.5, 0.5, size=(1, n)).astype(np.float16)
    expected_weight = (quantized.astype(np.float32) * scales.T.astype(np.float32)
                       + biases.T.astype(np.float32))
    expected = (activations.astype(np.float32) @ expected_weight.T).astype(np.float16)

    w_q = O.pack_codes(quantized, 4)
    got32 = O.affine_qmv(activations, w_q, scales.T.copy(), biases.T.copy(), 64, 4, dtype="f16",
                         acc=np.float32)
    np.testing.assert_array_equal(O.from_f32(got32.astype(np.float32), "f16"), expected)
    np.testing.assert_array_equal(O.dequantize(w_q, scales.T.copy(), biases.T.copy(), 64, 4,
                                               "f16"), expected_weight)


def test_qmv_matches_torch_cpu_independent_path():
    w_q, s, b = O.make_affine_weight(40, 512, 4, 64, config_id=1, tensor_id=10)
    x = O.make_activations(5, 512, config_id=1)
    got = O.affine_qmv(x, w_q, s, b, 64, 4)
    # torch: unpack with int64 shifts, dequantize, fp64 matmul
    wt = torch.from_numpy(w_q.astype(np.int64))
    shifts = torch.arange(0, 32, 4, dtype=torch.int64)
    q = ((wt[:, :, None] >> shifts) & 15).reshape(40, 512).double()
    st_ = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16).double()
    bt = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).double()
    w = q * st_.repeat_interleave(64, dim=1) + bt.repeat_interleave(64, dim=1)
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).double()
    np.testing.assert_allclose(got, (xt @ w.T).numpy(), rtol=1e-12, atol=1e-10)


# ---- SwiGLU / MLP -------------------------------------------------------------------------


def test_silu_mul_special_cases():
    g = np.array([0.0, 60.0, -60.0, 1.0, -1.0])
    u = np.array([3.0, 2.0, 2.0, 1.0, 1.0])
    out = O.silu_mul(g, u)
    assert out[0] == 0.0
    assert out[1] == pytest.approx(120.0)
    assert abs(out[2]) < 1e-20
    ref = torch.nn.functional.silu(torch.tensor(g)) * torch.tensor(u)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-12)
    with np.errstate(over="raise"):
        pass
    assert np.isfinite(O.silu_mul(np.array([-1e4]), np.array([1.0]))).all()


def test_mlp_composition_matches_torch_cpu():
    h, i, m = 128, 192, 3
    gate = O.make_affine_weight(i, h, 4, 64, 1, 10)
    up = O.make_affine_weight(i, h, 4, 64, 1, 12)
    down = O.make_affine_weight(h, i, 4, 64, 1, 14)
    x = O.make_activations(m, h, 1)
    res = O.make_activations(m, h, 1, tensor_id=3)
    y, hid = O.affine_mlp(x, gate, up, down, 64, 4, residual=res)

    def deq(t):
        return torch.from_numpy(O.dequantize(*t, 64, 4).astype(np.float64))

    xt = torch.from_numpy(O.bf16_bits_to_f32(x).astype(np.float64))
    hh = torch.nn.functional.silu(xt @ deq(gate).T) * (xt @ deq(up).T)
    hh_b = hh.float().to(torch.bfloat16)
    np.testing.assert_array_equal(hid, hh_b.view(torch.int16).numpy().view(np.uint16))
    yt = hh_b.double() @ deq(down).T + torch.from_numpy(O.bf16_bits_to_f32(res).astype(np.float64))
    np.testing.assert_allclose(y, yt.numpy(), rtol=1e-12, atol=1e-10)


# ---- dense typed rounding -----------------------------------------------------------------


def test_dense_swiglu_matches_torch_typed_ops():
    k, n, m = 256, 64, 4
    x = O.make_activations(m, k, 2)
    g = O.make_dense_weight(n, k, 2, 10)
    u = O.make_dense_weight(n, k, 2, 11)
    got = O.dense_swiglu(x, g, u)

    def tb(a):
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)

    xt = tb(x).double()
    left = (xt @ tb(g).double().T).float().to(torch.bfloat16)
    right = (xt @ tb(u).double().T).float().to(torch.bfloat16)
    y = 1 / (1 + torch.exp(left.abs()))          # each op rounds to bf16 on torch CPU
    sig = torch.where(left < 0, y, 1 - y)
    act = left * sig
    out = act * right
    np.testing.assert_array_equal(got, out.view(torch.int16).numpy().view(np.uint16))


def _dense_epilogue(left_bits, right_bits, fn=None):
    """Drive ``O.dense_swiglu`` with x = e0 (one 1.0), so that the gate and up dot products are
    exactly the given bf16 values and only the typed epilogue acts on them."""
    fn = fn or O.dense_swiglu
    n, k = left_bits.size, 64
    x = np.zeros((1, k), np.uint16)
    x[0, 0] = 0x3F80
    g = np.zeros((n, k), np.uint16)
    u = np.zeros((n, k), np.uint16)
    g[:, 0], u[:, 0] = left_bits, right_bits
    return fn(x, g, u)[0]


def _reversed_select(x, g, u):
    """A planted mistake: the sign select reversed (equivalently exp(-|g|) in place of
    exp(|g|)), i.e. g * sigmoid(-g) * u: the oracle applied to -g, negated."""
    return O.from_f32(-O.to_f32(O.dense_swiglu(x, O.from_f32(-O.to_f32(g, "bf16"), "bf16"), u),
                                "bf16"), "bf16")


def _bf16_grid(lo, hi):
    """Every finite bf16 value v with lo <= |v| <= hi, and zero (bit patterns, values)."""
    b = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    with np.errstate(invalid="ignore"):
        v = O.bf16_bits_to_f32(b).astype(np.float64)
    keep = np.isfinite(v) & (((np.abs(v) >= lo) & (np.abs(v) <= hi)) | (v == 0))
    return b[keep], v[keep]


U_SWEEP = [1.0, 1.5, -3.0, 0.0234375, 1.0078125, -0.7109375, 113.0]


def _ulps_from_exact(got_bits, exact):
    mag = np.maximum(np.abs(exact), 2.0 ** -126)
    ulp = np.ldexp(1.0, (np.floor(np.log2(mag)) - 7).astype(np.int64))
    return np.abs(O.bf16_bits_to_f32(got_bits).astype(np.float64) - exact) / ulp


def test_dense_swiglu_within_three_ulps_of_exact_silu_exhaustive():
    """Every bf16 gate value in [2^-100, 80] (and 0) against fp64 silu(g) * u for u values whose
    products land on bf16 rounding ties. The typed chain rounds six times (exp, 1 + e, the
    reciprocal, 1 - y, g * sig, act * u), each by at most half an ulp, and 1 - y (y <= 1/2)
    does not amplify y's error relative to the result, so it stays within 3 ulps of the exact
    value (measured maximum 2.6)."""
    left, lv = _bf16_grid(2.0 ** -100, 80.0)
    for uval in U_SWEEP:
        ub = O.f32_to_bf16_bits(np.full(left.size, uval, np.float32))
        exact = lv / (1.0 + np.exp(-lv)) * uval
        err = _ulps_from_exact(_dense_epilogue(left, ub), exact)
        assert err.max() <= 3.0, (uval, float(err.max()), float(lv[np.argmax(err)]))
        bad = _ulps_from_exact(_dense_epilogue(left, ub, _reversed_select), exact)
        assert bad.max() > 100.0, uval  # the planted mistake fails the same bound


def test_dense_swiglu_special_cases_zero_and_saturation():
    """g = 0 gives exactly 0; g >= 8 gives exactly round(g * u) (1 - y rounds to 1 once
    y < 2^-9, i.e. g > ln 511); g <= -89 gives exactly 0 (exp overflows, y = 0); for
    -89 < g <= -20 the result has the sign of -u and magnitude at most |g u| e^g (1 + 2^-6)."""
    for uval in U_SWEEP:
        left, lv = _bf16_grid(8.0, 1.0e30)
        pos = lv > 0
        left, lv = left[pos], lv[pos]
        ub = O.f32_to_bf16_bits(np.full(left.size, uval, np.float32))
        with np.errstate(over="ignore"):
            want = O.f32_to_bf16_bits((lv * uval).astype(np.float32))
        np.testing.assert_array_equal(_dense_epilogue(left, ub), want)
        assert not np.array_equal(_dense_epilogue(left, ub, _reversed_select), want)

        def us(count):
            return O.f32_to_bf16_bits(np.full(count, uval, np.float32))

        zero = np.array([0x0000, 0x8000], np.uint16)
        out = O.bf16_bits_to_f32(_dense_epilogue(zero, us(2)))
        np.testing.assert_array_equal(out, [0.0, 0.0])

        left, lv = _bf16_grid(89.0, 3.0e38)
        left = left[lv < 0]
        out = O.bf16_bits_to_f32(_dense_epilogue(left, us(left.size)))
        np.testing.assert_array_equal(out, np.zeros(left.size))

        left, lv = _bf16_grid(20.0, 88.9)
        neg = lv < 0
        left, lv = left[neg], lv[neg]
        out = O.bf16_bits_to_f32(_dense_epilogue(left, us(left.size))).astype(np.float64)
        bound = np.abs(lv * uval) * np.exp(lv) * (1 + 2.0 ** -6)
        assert np.all(np.abs(out) <= bound)
        assert np.all((out == 0) | (np.sign(out) == -np.sign(uval)))


def test_dense_swiglu_rounds_the_dot_products_before_the_epilogue():
    """g = 1 + 2^-8 + 2^-12 (a sum of exact products, not a bf16 value) must enter the epilogue
    as bf16(g) = 1 + 2^-7: the result equals the epilogue of 1 + 2^-7 exactly, and differs from
    that of 1.0 (the value a truncation would give)."""
    x = np.zeros((1, 64), np.uint16)
    x[0, :3] = O.f32_to_bf16_bits(np.array([1.0, 1.0, 1.0], np.float32))
    g = np.zeros((1, 64), np.uint16)
    g[0, :3] = O.f32_to_bf16_bits(np.array([1.0, 2.0 ** -8, 2.0 ** -12], np.float32))
    u = np.zeros((1, 64), np.uint16)
    u[0, 0] = 0x3FC0  # 1.5
    got = O.dense_swiglu(x, g, u)[0]
    up = O.f32_to_bf16_bits(np.array([1.0 + 2.0 ** -7], np.float32))
    one = O.f32_to_bf16_bits(np.array([1.0], np.float32))
    u1 = np.array([0x3FC0], np.uint16)
    assert got[0] == _dense_epilogue(up, u1)[0]
    assert got[0] != _dense_epilogue(one, u1)[0]


def _f32_dots_reversed(x, w):
    """fp32 dot products summed in reverse K order (another summation order than the oracle's
    fp64 one), as a GPU accumulation might give them."""
    xf = O.to_f32(x, "bf16")
    wf = O.to_f32(w, "bf16")
    acc = np.zeros((xf.shape[0], wf.shape[0]), np.float32)
    for k in range(xf.shape[1] - 1, -1, -1):
        acc += xf[:, k:k + 1] * wf[None, :, k]
    return acc


def test_budget_error_accepts_the_typed_chains_and_other_summation_orders():
    """The oracle's typed outputs score ~0 against the exact results with their rounding budget,
    and so do typed chains fed fp32 dot products summed in another order (which flip some
    intermediate roundings: a one-ulp flip of the output would be several 1e-3 of the typed
    reference, but scores only the accumulation noise here)."""
    k, n, m = 2048, 96, 4
    x = O.make_activations(m, k, 2)
    g = O.make_dense_weight(n, k, 2, 10)
    u = O.make_dense_weight(n, k, 2, 11)
    d = O.make_dense_weight(n, k, 2, 12)
    r = O.make_activations(m, n, 2, tensor_id=3)
    ex, bud = O.dense_swiglu_exact(x, g, u)
    assert O.budget_tolerance_error(O.dense_swiglu(x, g, u), ex, bud) <= 1e-9
    exr, budr = O.dense_residual_exact(x, d, r)
    assert O.budget_tolerance_error(O.dense_residual_qmv(x, d, r), exr, budr) <= 1e-9
    ex0, bud0 = O.dense_residual_exact(x, d, None)
    assert O.budget_tolerance_error(O.dense_residual_qmv(x, d, None), ex0, bud0) <= 1e-9

    left = O.f32_to_bf16_bits(_f32_dots_reversed(x, g))
    right = O.f32_to_bf16_bits(_f32_dots_reversed(x, u))
    typed = np.stack([_dense_epilogue(left[i], right[i]) for i in range(m)])
    assert O.budget_tolerance_error(typed, ex, bud) < 1e-5
    proj = O.bf16_bits_to_f32(O.f32_to_bf16_bits(_f32_dots_reversed(x, d)))
    typed_r = O.f32_to_bf16_bits(proj + O.bf16_bits_to_f32(r))
    assert O.budget_tolerance_error(typed_r, exr, budr) < 1e-5


def test_budget_error_over_every_bf16_gate_value():
    left, _ = _bf16_grid(2.0 ** -100, 80.0)
    for uval in U_SWEEP:
        ub = O.f32_to_bf16_bits(np.full(left.size, uval, np.float32))
        x = np.zeros((1, 64), np.uint16)
        x[0, 0] = 0x3F80
        gw = np.zeros((left.size, 64), np.uint16)
        uw = np.zeros((left.size, 64), np.uint16)
        gw[:, 0], uw[:, 0] = left, ub
        ex, bud = O.dense_swiglu_exact(x, gw, uw)
        assert O.budget_tolerance_error(O.dense_swiglu(x, gw, uw), ex, bud) <= 1e-9, uval


def test_budget_error_fails_planted_mistakes():
    k, n, m = 512, 64, 3
    x = O.make_activations(m, k, 2)
    g = O.make_dense_weight(n, k, 2, 10)
    u = O.make_dense_weight(n, k, 2, 11)
    r = O.make_activations(m, n, 2, tensor_id=3)
    ex, bud = O.dense_swiglu_exact(x, g, u)
    assert O.budget_tolerance_error(_reversed_select(x, g, u), ex, bud) > 2e-3
    assert O.budget_tolerance_error(O.dense_swiglu(x, g, u)[:, ::-1], ex, bud) > 2e-3
    exr, budr = O.dense_residual_exact(x, g, r)
    assert O.budget_tolerance_error(O.dense_residual_qmv(x, g, None), exr, budr) > 2e-3
    assert O.budget_tolerance_error(O.dense_residual_qmv(x, u, r), exr, budr) > 2e-3


def test_dense_residual_rounds_projection_then_sum():
    k, n, m = 128, 32, 3
    x = O.make_activations(m, k, 2)
    w = O.make_dense_weight(n, k, 2, 12)
    r = O.make_activations(m, n, 2, tensor_id=3)
    got = O.dense_residual_qmv(x, w, r)

    def tb(a):
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)

    proj = (tb(x).double() @ tb(w).double().T).float().to(torch.bfloat16)
    out = proj + tb(r)
    np.testing.assert_array_equal(got, out.view(torch.int16).numpy().view(np.uint16))


# ---- tolerance metric ---------------------------------------------------------------------


def test_tolerance_metric_catches_planted_mistakes():
    w_q, s, b = O.make_affine_weight(64, 512, 4, 64, 0, 1)
    x = O.make_activations(2, 512, 0)
    ref = O.affine_qmv(x, w_q, s, b, 64, 4)
    exact = O.from_f32(ref.astype(np.float32), "bf16")
    assert O.tolerance_error(exact, ref) == 0.0
    # dropped bias term
    no_bias = O.affine_qmv(x, w_q, s, np.zeros_like(b), 64, 4)
    assert O.tolerance_error(O.from_f32(no_bias.astype(np.float32), "bf16"), ref) > 1e-1
    # transposed / misindexed weight: shuffled output columns
    perm = O.from_f32(ref[:, ::-1].astype(np.float32), "bf16")
    assert O.tolerance_error(perm, ref) > 1e-1
    # one-ulp perturbation of a mid-size element stays within the contract
    bumped = exact.copy()
    bumped[0, 3] += 1
    assert O.tolerance_error(bumped, ref) < 2e-3 * 4


def test_algorithmic_bytes_config0():
    assert O.algorithmic_bytes_affine(1, 1536, 8960, 4, 64) == 7_762_432


# ---- affine quantization --------------------------------------------------------------------


def _group_row(values, group=32):
    """One row holding ``values`` tiled to a group, as bf16 storage."""
    v = np.resize(np.asarray(values, dtype=np.float32), group)
    return O.from_f32(v[None, :], "bf16")


def test_quantize_known_answer_ascending_ramp():
    w = _group_row(np.arange(16, dtype=np.float32))
    w_q, s, b = O.affine_quantize(w, 32, 4)
    assert O.to_f32(s, "bf16")[0, 0] == -1.0 and O.to_f32(b, "bf16")[0, 0] == 15.0
    codes = O.unpack_codes(w_q, 4)[0]
    np.testing.assert_array_equal(codes, 15 - np.resize(np.arange(16), 32))
    np.testing.assert_array_equal(O.dequantize(w_q, s, b, 32, 4), O.to_f32(w, "bf16"))


def test_quantize_known_answer_negative_ramp():
    w = _group_row(-np.arange(16, dtype=np.float32))
    w_q, s, b = O.affine_quantize(w, 32, 4)
    assert O.to_f32(s, "bf16")[0, 0] == 1.0 and O.to_f32(b, "bf16")[0, 0] == -15.0
    np.testing.assert_array_equal(O.dequantize(w_q, s, b, 32, 4), O.to_f32(w, "bf16"))


@pytest.mark.parametrize("c", [0.0, 0.375, -2.5])
def test_quantize_constant_groups_are_exact(c):
    w = _group_row([c])
    for bits in (4, 8):
        w_q, s, b = O.affine_quantize(w, 32, bits)
        np.testing.assert_array_equal(O.unpack_codes(w_q, bits), 0)
        np.testing.assert_array_equal(O.dequantize(w_q, s, b, 32, bits), O.to_f32(w, "bf16"))


@pytest.mark.parametrize("bits,g,dtype", [(4, 64, "bf16"), (8, 32, "bf16"), (4, 128, "f16")])
def test_quantize_reconstruction_and_brute_force(bits, g, dtype):
    rng = np.random.default_rng(bits * 1000 + g)
    w = O.from_f32((rng.standard_normal((6, 256)) * 0.02).astype(np.float32), dtype)
    w_q, s, b = O.affine_quantize(w, g, bits, dtype)
    wf = O.to_f32(w, dtype)
    deq = O.dequantize(w_q, s, b, g, bits, dtype)
    sf = np.repeat(np.abs(O.to_f32(s, dtype)), g, axis=1)
    # half a quantization step, plus what the 16-bit rounding of scale and bias can add; a
    # clamped code may be a full step off (the edge rule can round q0 away from the range, e.g.
    # max = -min gives q0 = rint(-7.5) = -8 at 4 bits and the other extreme maps to 16)
    ulp = 2.0 ** (-8 if dtype == "bf16" else -11)
    bf = np.repeat(np.abs(O.to_f32(b, dtype)), g, axis=1)
    extra = ((1 << bits) - 1) * sf * ulp + bf * ulp + 1e-12
    codes_all = O.unpack_codes(w_q, bits)
    inner = (codes_all > 0) & (codes_all < (1 << bits) - 1)
    err = np.abs(deq - wf)
    assert np.all(err[inner] <= (0.5 * sf + extra)[inner])
    assert np.all(err <= sf + extra)
    # brute force: the same rule written out per group with Python floats rounded to float32
    f32 = np.float32
    codes = O.unpack_codes(w_q, bits)
    for r in range(wf.shape[0]):
        for gi in range(wf.shape[1] // g):
            grp = wf[r, gi * g:(gi + 1) * g]
            hi, lo = f32(grp.max()), f32(grp.min())
            low = abs(lo) > abs(hi)
            sc = f32(max(f32(f32(hi - lo) / f32((1 << bits) - 1)), f32(1e-7)))
            sc = sc if low else f32(-sc)
            edge = lo if low else hi
            q0 = f32(np.rint(f32(edge / sc)))
            bias = f32(0)
            if q0 != 0:
                sc, bias = f32(edge / q0), edge
            s16 = O.to_f32(O.from_f32(np.array([sc], f32), dtype), dtype)[0]
            b16 = O.to_f32(O.from_f32(np.array([bias], f32), dtype), dtype)[0]
            assert O.to_f32(s, dtype)[r, gi] == s16 and O.to_f32(b, dtype)[r, gi] == b16
            want = [min(max(np.rint(f32(f32(v - b16) / s16)), 0), (1 << bits) - 1) for v in grp]
            np.testing.assert_array_equal(codes[r, gi * g:(gi + 1) * g], want)
