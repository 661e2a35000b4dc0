"""NumPy restatement of meTile's affine quantized-projection arithmetic (TEST INFRASTRUCTURE ONLY).

This module is the checker for the HIP kernels in ``metile_amd``. It is imported only by
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg; the product
path never calls it.

Every function cites the reference lines it restates (paths under the meTile source tree).
How each function is pinned (known answers, closed forms, brute force, an independent
implementation) is listed in ``PINNED_BY`` at the bottom of this file and exercised by
``tests/test_oracle.py``.

Storage conventions (MLX affine format, as consumed by the reference kernels):

* ``w_q``: uint32 ``[N, K*bits/32]``, output-major; code ``k`` of row ``n`` sits in word
  ``k // (32//bits)`` at bit offset ``(k % (32//bits)) * bits`` (low bits first along K).
  ``kernels/affine_qmv.py:25-27,40-47``; ``metile/backends/mlx_quantized.py:768-770``.
* ``scales``, ``biases``: ``[N, K/group_size]`` in the activation dtype.
  ``metile/backends/mlx_quantized.py:1556-1565``.
* bf16 tensors are carried as ``uint16`` bit patterns so that rounding is explicit.
"""

from __future__ import annotations

import numpy as np

# --------------------------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even written against the uint32 bit pattern)
# --------------------------------------------------------------------------------------------


def f32_to_bf16_bits(values) -> np.ndarray:
    """Round float32 values to bf16 (RNE) and return the uint16 bit patterns.

    NaNs stay NaN (quietened); infinities and signed zeros are preserved.
    """
    f = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    rounded = (u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)
    nan = np.isnan(f)
    out = rounded.astype(np.uint16)
    if nan.any():
        out = np.where(nan, ((u >> np.uint64(16)) | np.uint64(0x40)).astype(np.uint16), out)
    return out


def bf16_bits_to_f32(bits) -> np.ndarray:
    """Widen bf16 bit patterns (uint16) to float32 exactly."""
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(values) -> np.ndarray:
    """Round to the nearest bf16 value (RNE) and return it as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(values))


def to_f32(values, dtype: str) -> np.ndarray:
    """Interpret activation-dtype storage as float32: bf16 from uint16 bits, f16/f32 natively."""
    if dtype == "bf16":
        return bf16_bits_to_f32(values)
    return np.asarray(values).astype(np.float32)


def from_f32(values, dtype: str) -> np.ndarray:
    """Round float32 values into activation-dtype storage (bf16 as uint16 bits, RNE)."""
    if dtype == "bf16":
        return f32_to_bf16_bits(values)
    if dtype == "f16":
        return np.asarray(values, dtype=np.float32).astype(np.float16)
    return np.asarray(values, dtype=np.float32)


def half_ulp(values, dtype: str = "bf16") -> np.ndarray:
    """Half a unit in the last place of ``values`` in ``dtype`` (the RNE output-rounding bound)."""
    v = np.abs(np.asarray(values, dtype=np.float64))
    mant = {"bf16": 7, "f16": 10, "f32": 23}[dtype]
    min_exp = {"bf16": -126, "f16": -14, "f32": -126}[dtype]
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(v > 0, v, 1.0)))
    e = np.maximum(e, min_exp)
    return np.ldexp(1.0, (e - mant - 1).astype(np.int64))


# --------------------------------------------------------------------------------------------
# Packing format
# --------------------------------------------------------------------------------------------


def pack_codes(codes, bits: int) -> np.ndarray:
    """Pack integer codes ``[N, K]`` into MLX affine uint32 words ``[N, K*bits/32]``.

    Code ``k`` goes to word ``k // (32//bits)`` at shift ``(k % (32//bits)) * bits``.
    Restates the layout read by ``kernels/affine_qmv.py:40-47`` (word index along K, shift
    ``element * BITS``) and produced/consumed by ``metile/backends/mlx_quantized.py:768-770``.
    """
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    c = np.asarray(codes)
    if c.ndim != 2:
        raise ValueError("codes must be [N, K]")
    per_word = 32 // bits
    n, k = c.shape
    if k % per_word:
        raise ValueError("K must be a multiple of 32/bits")
    if c.size and (c.min() < 0 or c.max() >= (1 << bits)):
        raise ValueError("codes out of range")
    c = c.astype(np.uint32).reshape(n, k // per_word, per_word)
    shifts = (np.arange(per_word, dtype=np.uint32) * np.uint32(bits))[None, None, :]
    return np.bitwise_or.reduce(c << shifts, axis=2).astype(np.uint32)


def unpack_codes(w_q, bits: int) -> np.ndarray:
    """Unpack MLX affine uint32 words ``[N, W]`` into codes ``[N, W*32/bits]`` (uint32).

    Restates ``(packed >> (element * BITS)) & ((1 << BITS) - 1)`` from
    ``kernels/affine_qmv.py:45-47``.
    """
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    w = np.asarray(w_q, dtype=np.uint32)
    per_word = 32 // bits
    shifts = (np.arange(per_word, dtype=np.uint32) * np.uint32(bits))[None, None, :]
    codes = (w[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
    return codes.reshape(w.shape[0], w.shape[1] * per_word)


def repack_step_major(w_q, bits: int) -> np.ndarray:
    """Step-major repack of MLX affine words ``[N, K*bits/32]`` into ``[K/64, N, 2*bits]``
    words: chunk ``[t, n]`` holds the ``8*bits`` bytes of row ``n`` that carry codes
    ``[64t, 64t + 64)``, unchanged. This is the layout the gfx950 small-row kernels read; it has
    no counterpart in the reference, whose repack (``metile/backends/mlx_quantized.py:754-774``)
    produces a K-major nibble layout for its NAX kernels. A pure reordering of whole 32-bit
    words (a 64-code chunk is 2*bits words), written as a reshape and transpose.
    """
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    w = np.ascontiguousarray(np.asarray(w_q, dtype=np.uint32))
    n, words = w.shape
    chunk = 2 * bits  # words per 64 codes
    if words % chunk:
        raise ValueError("K must be a multiple of 64")
    return np.ascontiguousarray(w.reshape(n, words // chunk, chunk).transpose(1, 0, 2))


def affine_quantize(w, group_size: int, bits: int, dtype: str = "bf16"):
    """Affine group quantization of dense 16-bit weights ``[N, K]`` (storage of ``dtype``) into
    ``(w_q, scales, biases)`` in the MLX affine format, all arithmetic in float32.

    Restates MLX's published affine quantize (``mx.quantize(w, group_size, bits,
    mode="affine")``, mlx 0.32, called by ``metile/backends/mlx_compressed_down.py:41-48``):
    per group, ``scale = max((max - min) / (2^bits - 1), 1e-7)``, negated unless
    ``|min| > |max|``; the extreme of larger magnitude (``edge``) is made exactly representable:
    ``q0 = rint(edge / scale)``, and if ``q0 != 0`` then ``scale = edge / q0`` and
    ``bias = edge``, else ``bias = 0``. Scale and bias are rounded to ``dtype``; the codes are
    ``rint((w - bias) / scale)`` with the rounded values, clamped to ``[0, 2^bits - 1]``.
    Parity with MLX itself is unpinned (MLX is not installed); the known answers and bounds in
    ``PINNED_BY`` pin this restatement.
    """
    wf = to_f32(w, dtype)
    n, k = wf.shape
    if k % group_size:
        raise ValueError("K must be a multiple of group_size")
    g = wf.reshape(n, k // group_size, group_size)
    bins = np.float32((1 << bits) - 1)
    w_max = g.max(axis=-1)
    w_min = g.min(axis=-1)
    low = np.abs(w_min) > np.abs(w_max)
    scale = np.maximum((w_max - w_min) / bins, np.float32(1e-7)).astype(np.float32)
    scale = np.where(low, scale, -scale).astype(np.float32)
    edge = np.where(low, w_min, w_max).astype(np.float32)
    q0 = np.rint(edge / scale).astype(np.float32)
    nonzero = q0 != 0
    scale = np.where(nonzero, edge / np.where(nonzero, q0, np.float32(1)), scale)
    bias = np.where(nonzero, edge, np.float32(0)).astype(np.float32)
    s_store = from_f32(scale.astype(np.float32), dtype)
    b_store = from_f32(bias, dtype)
    s = to_f32(s_store, dtype)[..., None]
    b = to_f32(b_store, dtype)[..., None]
    codes = np.clip(np.rint((g - b) / s), 0, bins).astype(np.uint32).reshape(n, k)
    return pack_codes(codes, bits), s_store, b_store


def dequantize(w_q, scales, biases, group_size: int, bits: int, dtype: str = "bf16") -> np.ndarray:
    """Exact fp32 dequantization ``w = q*s + b`` with per-(row, group) scale and bias.

    Restates ``quantized * scale + bias`` of ``kernels/affine_qmv.py:41-51`` with the f32
    decode dtype (``decode_dtype="f32"``, ``metile/backends/mlx_quantized.py:691-714``).
    The product ``q*s`` is exact in fp32 (q < 2^8, s has an 8- or 11-bit significand), so the
    single fp32 rounding happens in the add; FMA and mul+add give the same bits.
    """
    q = unpack_codes(w_q, bits).astype(np.float32)
    n, k = q.shape
    if k % group_size:
        raise ValueError("K must be a multiple of group_size")
    s = to_f32(scales, dtype).reshape(n, k // group_size)
    b = to_f32(biases, dtype).reshape(n, k // group_size)
    s_full = np.repeat(s, group_size, axis=1)
    b_full = np.repeat(b, group_size, axis=1)
    return (q * s_full + b_full).astype(np.float32)


# --------------------------------------------------------------------------------------------
# Projections
# --------------------------------------------------------------------------------------------


def affine_qmv(x, w_q, scales, biases, group_size: int, bits: int, *, residual=None,
               dtype: str = "bf16", acc=np.float64) -> np.ndarray:
    """Unrounded ``y[m, n] = sum_k x[m, k] * (q[n, k]*s + b) (+ residual[m, n])``.

    Restates ``_affine_qmv_results`` (``kernels/affine_qmv.py:4-54``) and the residual epilogue
    ``results + residual`` (``kernels/affine_qmv.py:124-132``); the semantic reference is
    ``mx.quantized_matmul(x, w, scales, biases, transpose=True)``
    (``metile/backends/mlx_quantized.py:834-855``). ``acc`` selects the accumulation type
    (float64 for the exact reference, float32 for the fp32-accumulated reference).
    Returns float64 values over leading dims ``x.shape[:-1]``.
    """
    xf = to_f32(x, dtype)
    lead = xf.shape[:-1]
    x2 = xf.reshape(-1, xf.shape[-1]).astype(acc)
    w = dequantize(w_q, scales, biases, group_size, bits, dtype).astype(acc)
    y = x2 @ w.T
    if residual is not None:
        y = y + to_f32(residual, dtype).reshape(y.shape).astype(acc)
    return y.astype(np.float64).reshape(*lead, w.shape[0])


def silu_mul(gate, up) -> np.ndarray:
    """``gate / (1 + exp(-gate)) * up`` in float64, the fused epilogue of
    ``kernels/affine_qmv.py:208`` (also ``nn.silu(g) * u``,
    ``metile/backends/mlx_quantized.py:917``)."""
    g = np.asarray(gate, dtype=np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g)) * np.asarray(up, dtype=np.float64)


def affine_swiglu(x, gate, up, group_size: int, bits: int, *, dtype: str = "bf16",
                  acc=np.float64) -> np.ndarray:
    """Unrounded fused SwiGLU ``silu(x @ Wg^T) * (x @ Wu^T)``; ``gate``/``up`` are
    ``(w_q, scales, biases)`` triples. Restates ``affine_swiglu_qmv``
    (``kernels/affine_qmv.py:135-214``): both dots accumulate in fp32 from one activation load
    and the SwiGLU is applied to the unrounded sums before a single store rounding."""
    g = affine_qmv(x, *gate, group_size, bits, dtype=dtype, acc=acc)
    u = affine_qmv(x, *up, group_size, bits, dtype=dtype, acc=acc)
    return silu_mul(g, u)


def affine_mlp(x, gate, up, down, group_size: int, bits: int, *, residual=None,
               dtype: str = "bf16", acc=np.float64):
    """``down(swiglu(x)) (+ residual)`` with the hidden activation rounded to ``dtype``.

    Restates ``mlx_affine_mlp_executor``'s ``residual_executor(swiglu_executor(values),
    residual)`` (``metile/backends/mlx_quantized.py:1770-1832``): the SwiGLU kernel stores its
    output in the activation dtype (``kernels/affine_qmv.py:209-214``) and the down projection
    reads it back. Returns ``(y_unrounded, h_storage)``.
    """
    h = from_f32(affine_swiglu(x, gate, up, group_size, bits, dtype=dtype, acc=acc), dtype)
    y = affine_qmv(h, *down, group_size, bits, residual=residual, dtype=dtype, acc=acc)
    return y, h


def affine_matmul(x, w_q, scales, biases, group_size: int, bits: int, *, dtype: str = "bf16",
                  acc=np.float64) -> np.ndarray:
    """Prefill affine GEMM semantics: the same sum as :func:`affine_qmv` for many rows.

    Restates ``_native_affine_matmul`` (``metile/backends/mlx_affine.py:142-154``): an affine
    ``quantized_matmul`` with ``transpose=True`` over row-major activations.
    """
    return affine_qmv(x, w_q, scales, biases, group_size, bits, dtype=dtype, acc=acc)


# --------------------------------------------------------------------------------------------
# Dense BF16 small-batch SwiGLU (typed rounding points)
# --------------------------------------------------------------------------------------------


def dense_swiglu(x, gate_w, up_w, *, dtype: str = "bf16") -> np.ndarray:
    """Dense SwiGLU with the reference's typed epilogue; returns ``dtype`` storage.

    Restates ``_emit_paired_dot_swiglu_store`` (``metile/codegen/msl_emitter.py:1218-1252``)
    with ``round_intermediates="half"`` specialised to the activation type
    (``metile/compiler/dense.py:293-294``; ``metile/backends/mlx.py:150-171``): the fp32 dots
    are rounded to the activation type, then ``y = 1/(1+exp(|g|))``,
    ``sig = g < 0 ? y : 1 - y``, ``act = g*sig`` and ``out = act*u``, each operation rounded to
    the activation type (MLX's typed ``silu`` arithmetic). Accumulation is fp32-exact here
    (float64), so only the epilogue rounding points are restated.
    """
    xf = to_f32(x, dtype).astype(np.float64)
    lead = xf.shape[:-1]
    x2 = xf.reshape(-1, xf.shape[-1])
    g = x2 @ to_f32(gate_w, dtype).astype(np.float64).T
    u = x2 @ to_f32(up_w, dtype).astype(np.float64).T

    def r(v):
        return to_f32(from_f32(np.asarray(v, dtype=np.float32), dtype), dtype).astype(np.float64)

    left = r(g)
    right = r(u)
    with np.errstate(over="ignore"):
        e = r(np.exp(np.abs(left)))
    y = r(1.0 / r(1.0 + e))
    sig = np.where(left < 0, y, r(1.0 - y))
    act = r(left * sig)
    out = from_f32((act * right).astype(np.float32), dtype)
    return out.reshape(*lead, out.shape[-1])


def dense_residual_qmv(x, w, residual=None, *, dtype: str = "bf16") -> np.ndarray:
    """Dense down projection: ``out = T(T(acc) + residual)`` in storage dtype ``T``.

    Restates ``_emit_dot_residual_store`` (``metile/codegen/msl_emitter.py:1098-1120``): the
    projected value is rounded to the activation type before the residual add, and the sum is
    rounded again. Without a residual the output is ``T(acc)``.
    """
    xf = to_f32(x, dtype).astype(np.float64)
    lead = xf.shape[:-1]
    acc = xf.reshape(-1, xf.shape[-1]) @ to_f32(w, dtype).astype(np.float64).T
    projected = to_f32(from_f32(acc.astype(np.float32), dtype), dtype)
    if residual is None:
        out = from_f32(projected, dtype)
    else:
        res = to_f32(residual, dtype).reshape(projected.shape)
        out = from_f32((projected.astype(np.float64) + res).astype(np.float32), dtype)
    return out.reshape(*lead, out.shape[-1])


def dense_swiglu_exact(x, gate_w, up_w, *, dtype: str = "bf16"):
    """``(exact, budget)`` for the dense typed SwiGLU: ``exact`` = fp64 ``silu(g) * u`` of the
    exact dot products (no rounding anywhere), ``budget`` = the rounding error the reference's
    typed chain itself may spend at each output, to first order: the rounding of g and of u to
    the activation type carried through ``g -> silu(g) u`` (``|silu'(g) u|`` and ``|silu(g)|``
    times half an ulp of each), plus the epilogue's own six roundings, which stay within 3 ulps
    of the result (the bound ``tests/test_oracle.py`` pins over every bf16 gate value)."""
    xf = to_f32(x, dtype).astype(np.float64)
    lead = xf.shape[:-1]
    x2 = xf.reshape(-1, xf.shape[-1])
    g = x2 @ to_f32(gate_w, dtype).astype(np.float64).T
    u = x2 @ to_f32(up_w, dtype).astype(np.float64).T
    with np.errstate(over="ignore"):
        sig = 1.0 / (1.0 + np.exp(-g))
    exact = g * sig * u
    dsilu = sig * (1.0 + g * (1.0 - sig))
    budget = (half_ulp(g, dtype) * np.abs(dsilu * u) + half_ulp(u, dtype) * np.abs(g * sig)
              + 6.0 * half_ulp(exact, dtype))
    return exact.reshape(*lead, -1), budget.reshape(*lead, -1)


def dense_residual_exact(x, w, residual=None, *, dtype: str = "bf16"):
    """``(exact, budget)`` for ``T(T(x @ w^T) + residual)``: ``exact`` = fp64 ``acc + residual``,
    ``budget`` = half an ulp of ``acc`` (its rounding to T) plus half an ulp of the sum at the
    largest magnitude the rounded projection can give it (without a residual: half an ulp of
    ``acc``)."""
    xf = to_f32(x, dtype).astype(np.float64)
    lead = xf.shape[:-1]
    acc = xf.reshape(-1, xf.shape[-1]) @ to_f32(w, dtype).astype(np.float64).T
    h_acc = half_ulp(acc, dtype)
    if residual is None:
        return acc.reshape(*lead, -1), h_acc.reshape(*lead, -1)
    exact = acc + to_f32(residual, dtype).astype(np.float64).reshape(acc.shape)
    budget = h_acc + half_ulp(np.abs(exact) + h_acc, dtype)
    return exact.reshape(*lead, -1), budget.reshape(*lead, -1)


# --------------------------------------------------------------------------------------------
# Tolerance
# --------------------------------------------------------------------------------------------


def tolerance_error(y_storage, ref, dtype: str = "bf16") -> float:
    """Max-abs-normalised error of a rounded output against an unrounded reference, after
    removing the unavoidable final RNE rounding to ``dtype``:

    ``max_i max(0, |y_i - ref_i| - half_ulp(ref_i)) / max_i |ref_i|``.

    The contract is ``<= 2e-3``. An exactly-rounded output scores 0; a one-ulp flip caused by
    accumulation noise near a rounding midpoint scores about the noise. Non-finite outputs
    score ``inf``.
    """
    y = to_f32(y_storage, dtype).astype(np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    if not np.all(np.isfinite(y)):
        return float("inf")
    scale = np.max(np.abs(r)) if r.size else 0.0
    if scale == 0.0:
        return float(np.max(np.abs(y))) if y.size else 0.0
    excess = np.maximum(np.abs(y - r) - half_ulp(r, dtype), 0.0)
    return float(np.max(excess) / scale)


def budget_tolerance_error(y_storage, exact, budget, dtype: str = "bf16") -> float:
    """The contract's max-abs-normalised error for outputs whose reference semantics round at
    intermediate points (the dense typed chains): ``max_i max(0, |y_i - exact_i| - budget_i) /
    max_i |exact_i|``, where ``exact`` is the unrounded fp64 result and ``budget`` the rounding
    error the reference's own roundings may spend (``dense_*_exact``). What remains is the
    error of the computation itself (its accumulation), which the contract bounds by 2e-3. An
    fp32 accumulation that lands on the other side of an intermediate rounding point than the
    exact sum scores about its own noise, not an ulp of the output. Non-finite outputs score
    ``inf``."""
    y = to_f32(y_storage, dtype).astype(np.float64).ravel()
    e = np.asarray(exact, dtype=np.float64).ravel()
    if not np.all(np.isfinite(y)):
        return float("inf")
    scale = np.max(np.abs(e)) if e.size else 0.0
    excess = np.maximum(np.abs(y - e) - np.asarray(budget, dtype=np.float64).ravel(), 0.0)
    if scale == 0.0:
        return float(np.max(excess)) if e.size else 0.0
    return float(np.max(excess) / scale)


def plain_error(y_storage, ref, dtype: str = "bf16") -> float:
    """``max|y - ref| / max|ref|`` including output rounding (reported, not the gate)."""
    y = to_f32(y_storage, dtype).astype(np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    scale = np.max(np.abs(r)) if r.size else 1.0
    return float(np.max(np.abs(y - r)) / (scale or 1.0)) if r.size else 0.0


# --------------------------------------------------------------------------------------------
# Seeded synthetic inputs
# --------------------------------------------------------------------------------------------


def rng(config_id: int, tensor_id: int) -> np.random.Generator:
    """One generator per tensor: ``default_rng(SeedSequence([config_id, tensor_id]))``."""
    return np.random.default_rng(np.random.SeedSequence([config_id, tensor_id]))


def make_activations(rows: int, k: int, config_id: int, tensor_id: int = 0,
                     dtype: str = "bf16") -> np.ndarray:
    """``x ~ N(0, 1)`` rounded (RNE) to the activation dtype."""
    return from_f32(rng(config_id, tensor_id).standard_normal((rows, k), dtype=np.float32), dtype)


def make_affine_weight(n: int, k: int, bits: int, group_size: int, config_id: int,
                       tensor_id: int, dtype: str = "bf16"):
    """BASELINE recipe: codes uniform in ``[0, 2^bits)``, ``scale = |N(0,1)| * c`` rounded to
    the dtype (c = 0.02 for 4-bit, 0.002 for 8-bit), ``bias = -zero * scale`` with zero = 8 or
    128 (exact: a power-of-two multiple). Returns ``(w_q, scales, biases)``."""
    codes = rng(config_id, tensor_id).integers(0, 1 << bits, size=(n, k), dtype=np.uint32)
    coef = 0.02 if bits == 4 else 0.002
    zero = 8.0 if bits == 4 else 128.0
    s32 = np.abs(rng(config_id, tensor_id + 1).standard_normal((n, k // group_size),
                                                                dtype=np.float32)) * np.float32(coef)
    scales = from_f32(s32, dtype)
    biases = from_f32(-zero * to_f32(scales, dtype), dtype)
    return pack_codes(codes, bits), scales, biases


def make_dense_weight(n: int, k: int, config_id: int, tensor_id: int,
                      dtype: str = "bf16") -> np.ndarray:
    """Dense weight ``N(0, 0.02)`` rounded to the activation dtype, ``[N, K]``."""
    return from_f32(rng(config_id, tensor_id).standard_normal((n, k), dtype=np.float32)
                    * np.float32(0.02), dtype)


def algorithmic_bytes_affine(m: int, k: int, n: int, bits: int, group_size: int,
                             act_bytes: int = 2, residual: bool = False) -> int:
    """Bytes one affine projection must move: packed weights, scales and biases, x in, y out
    (and the residual when fused)."""
    w = n * k * bits // 8 + 2 * act_bytes * n * (k // group_size)
    return w + act_bytes * m * k + act_bytes * m * n * (2 if residual else 1)


PINNED_BY = {
    "f32_to_bf16_bits": "exhaustive comparison with torch.bfloat16 casting on edge patterns",
    "pack_codes/unpack_codes": "hand-built words (0x76543210 -> 0..7), round trip (hypothesis)",
    "repack_step_major": "hand-built rows of known codes land at [t, n]; brute-force index loop; "
                         "the inverse transpose restores the words",
    "dequantize": "closed form (q - zero) * s, brute-force loop of kernels/affine_qmv.py:32-51",
    "affine_quantize": "known answers (a 0..15 ramp -> scale -1, bias 15; its negation -> scale "
                       "1, bias -15; constant and zero groups reproduced exactly); every element "
                       "within half a step of its dequantized value; brute-force per-group loop",
    "affine_qmv": "reference KAT tests/test_affine_quantized.py:120-163 (seed 211), torch CPU",
    "silu_mul": "special cases g=0, g>>0, g<<0, and torch.nn.functional.silu",
    "affine_mlp": "composition of pinned parts; torch CPU end-to-end",
    "dense_swiglu": "exhaustive bf16 gate sweep within 3 ulps of fp64 silu(g)*u (u on rounding "
                    "ties); g=0 -> 0, g>=8 -> round(g*u), g<=-89 -> 0, -89<g<=-20 bounded by "
                    "|g u| e^g; dot products rounded before the epilogue; a reversed sign "
                    "select fails these; torch CPU typed ops agree bit for bit",
    "dense_residual_qmv": "torch CPU (bf16 round of fp32 dot, then bf16 add)",
    "tolerance_error": "planted mistakes (dropped bias term, transposed weight) fail it",
    "dense_swiglu_exact/dense_residual_exact/budget_tolerance_error": "the oracle's own typed "
        "outputs score <= 1e-9 at config-2 magnitudes and over every bf16 gate value; typed "
        "chains fed fp32 dot products in another summation order score < 1e-5; a reversed sign "
        "select, a dropped residual and permuted outputs score > 2e-3",
}
