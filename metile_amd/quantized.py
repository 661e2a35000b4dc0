"""Affine quantized projections on torch tensors, backed by the gfx950 HIP kernels.

The public functions keep meTile's MLX-backend call surface
(``metile/backends/mlx_quantized.py``): the same names, positional/keyword arguments,
argument meaning and ``ValueError`` guards, but they take and return torch tensors on a ROCm
device and always run the hand-written HIP kernels through the C ABI. There is no fallback
path: the reference's ``autotune`` arguments choose among this library's own plans for a shape
(split-K, strips, kernel; ``metile_amd.tuning``), never another implementation.

Tensor formats (MLX affine): ``weight`` uint32 (or int32 holding the same bits)
``[N, K*bits/32]``; ``scales``/``biases`` ``[N, K/group_size]`` in the activation dtype
(bfloat16 or float16); activations ``[..., K]``. ``affine_qmv``, ``affine_swiglu`` and
``affine_mlp`` also take codes repacked ahead of time by ``affine_repack`` (step-major
``[K/64, N, 2*bits]``; the layout is told apart by the number of dimensions) and then give the
same results bit for bit.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass

import torch

from . import _lib
from . import tuning as _tuning

_DTYPES = {torch.bfloat16: _lib.MT_BF16, torch.float16: _lib.MT_F16}

# ---------------------------------------------------------------------------------------------
# workspace cache: one zero-initialised buffer per (device, stream), grown on demand
# ---------------------------------------------------------------------------------------------

_ws_lock = threading.RLock()
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
# Buffers replaced by a larger one stay allocated: a HIP graph captured earlier keeps their
# address. Growth doubles, so the retired buffers never exceed the live one.
_retired: list[torch.Tensor] = []


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(device: torch.device) -> int:
    """The current HIP stream of ``device`` as an integer handle (torch's raw getter when it has
    one: it builds no Stream object, about a microsecond less per call)."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def workspace(device: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor:
    """Return a zero-initialised uint8 workspace of at least ``nbytes`` for the current stream.

    Calls on one stream are ordered, so they may share it; the kernels leave its counter
    region zeroed after each call. ``stream``: the current stream's handle, if the caller has it. A buffer that is outgrown is kept, not freed, so that graphs
    captured over it stay valid.

    A buffer is never created or grown during graph capture: its zero fill would only be
    recorded into that graph, not run, and a later call or graph on the stream would find it
    uninitialised. Run the call once on the capturing stream, outside capture, first.
    """
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           _stream_handle(device) if stream is None else stream)
    with _ws_lock:
        buf = _workspaces.get(key)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "metile_amd: this stream has no workspace large enough for the call; run it "
                    "once on the capturing stream outside graph capture before capturing it")
            size = max(nbytes, 1 << 20, 2 * buf.numel() if buf is not None else 0)
            if buf is not None:
                _retired.append(buf)
            buf = torch.zeros(size, dtype=torch.uint8, device=device)
            _workspaces[key] = buf
        return buf


def _ptr(t):
    return None if t is None else t.data_ptr()


def _require_device(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("metile_amd operators take ROCm device tensors")


def _as_u32(weight: torch.Tensor) -> torch.Tensor:
    if weight.dtype not in (torch.uint32, torch.int32):
        raise ValueError("packed affine weights must be uint32 (or int32 holding the same bits)")
    return weight.contiguous()


def _dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise ValueError("activations must be bfloat16 or float16") from None


def _repacked(weight) -> bool:
    """Codes in the step-major repack of ``affine_repack`` rather than MLX's rows."""
    return weight.ndim == 3


def _layout_code(weight) -> int:
    return _lib.MT_LAYOUT_REPACKED if _repacked(weight) else _lib.MT_LAYOUT_MLX


def _code_shape(weight, bits):
    """``(N, K)`` of packed codes in either layout, or ``None`` if the shape is neither."""
    if weight.ndim == 2:
        return weight.shape[0], weight.shape[1] * 32 // bits
    if weight.ndim == 3 and weight.shape[2] == 2 * bits:
        return weight.shape[1], weight.shape[0] * 64
    return None


def _check_params(values, weight, scales, biases, group_size, bits, what):
    k = values.shape[-1]
    shape = _code_shape(weight, bits)
    if (shape is None or shape[1] != k
            or tuple(scales.shape) != (shape[0], k // group_size)
            or tuple(biases.shape) != (shape[0], k // group_size)):
        raise ValueError(f"{what} received incompatible quantization parameters")
    if scales.dtype != values.dtype or biases.dtype != values.dtype:
        raise ValueError(f"{what} parameters must match the input dtype")


# ---------------------------------------------------------------------------------------------
# general entry points
# ---------------------------------------------------------------------------------------------


def affine_qmv(values, weight, scales, biases, *, group_size=64, bits=4, residual=None):
    """``values @ dequantize(weight).T (+ residual)`` with fp32 accumulation.

    Semantics of ``mx.quantized_matmul(values, weight, scales, biases, transpose=True)`` as
    restated by ``kernels/affine_qmv.py:4-132``. Any leading shape; bits 4 or 8; group_size a
    multiple of 64 dividing K.
    """
    if biases is None:
        raise ValueError("affine QMV requires affine quantization biases")
    _require_device(values, weight, scales, biases, residual)
    code = _dtype_code(values.dtype)
    _check_params(values, weight, scales, biases, group_size, bits, "affine QMV")
    k = values.shape[-1]
    n = _code_shape(weight, bits)[0]
    lead = tuple(values.shape[:-1])
    x = values.reshape(-1, k).contiguous()
    m = x.shape[0]
    out = torch.empty(*lead, n, dtype=values.dtype, device=values.device)
    if m == 0:
        return out
    res = None
    if residual is not None:
        if tuple(residual.shape) != (*lead, n) or residual.dtype != values.dtype:
            raise ValueError("residual must match the affine QMV output shape and dtype")
        res = residual.reshape(m, n).contiguous()
    w = _as_u32(weight)
    s = scales.contiguous()
    b = biases.contiguous()
    L = _lib.lib()
    need = L.mt_affine_qmv_workspace_bytes(m, k, n, group_size, bits, 1)
    ws = workspace(values.device, need) if need else None
    fn = L.mt_affine_qmv_repacked if _repacked(w) else L.mt_affine_qmv
    _lib.check(fn(
        x.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(), _ptr(res), out.data_ptr(),
        m, k, n, group_size, bits, code, _ptr(ws), 0 if ws is None else ws.numel(),
        _stream_handle(values.device)))
    return out


def affine_swiglu(values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                  up_biases, *, group_size=64, bits=4):
    """Fused ``silu(values @ Wg^T) * (values @ Wu^T)``; gate and up stay in fp32 registers and
    are combined before the single output rounding (``kernels/affine_qmv.py:135-214``)."""
    if gate_biases is None or up_biases is None:
        raise ValueError("affine SwiGLU requires affine quantization biases")
    _require_device(values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                    up_biases)
    code = _dtype_code(values.dtype)
    if (gate_weight.shape != up_weight.shape or gate_scales.shape != up_scales.shape
            or gate_biases.shape != up_biases.shape or up_scales.dtype != values.dtype
            or up_biases.dtype != values.dtype):
        raise ValueError("affine SwiGLU requires matching gate/up weights and parameters")
    _check_params(values, gate_weight, gate_scales, gate_biases, group_size, bits, "affine SwiGLU")
    k = values.shape[-1]
    n = _code_shape(gate_weight, bits)[0]
    lead = tuple(values.shape[:-1])
    x = values.reshape(-1, k).contiguous()
    m = x.shape[0]
    out = torch.empty(*lead, n, dtype=values.dtype, device=values.device)
    if m == 0:
        return out
    gw, uw = _as_u32(gate_weight), _as_u32(up_weight)
    gs, gb = gate_scales.contiguous(), gate_biases.contiguous()
    us, ub = up_scales.contiguous(), up_biases.contiguous()
    L = _lib.lib()
    need = L.mt_affine_qmv_workspace_bytes(m, k, n, group_size, bits, 2)
    ws = workspace(values.device, need) if need else None
    fn = L.mt_affine_swiglu_repacked if _repacked(gw) else L.mt_affine_swiglu
    _lib.check(fn(
        x.data_ptr(), gw.data_ptr(), gs.data_ptr(), gb.data_ptr(), uw.data_ptr(), us.data_ptr(),
        ub.data_ptr(), out.data_ptr(), m, k, n, group_size, bits, code, _ptr(ws),
        0 if ws is None else ws.numel(), _stream_handle(values.device)))
    return out


def affine_mlp(values, gate, up, down, *, group_size=64, bits=4, residual=None):
    """``down(swiglu(values)) (+ residual)`` through one C-ABI call: the fused gate/up SwiGLU
    launch, then the down projection (with the residual epilogue) over the hidden activation,
    which stays in the workspace.

    ``gate``/``up``/``down`` are ``(weight, scales, biases)`` triples; gate/up ``[I, H]``,
    down ``[H, I]``, gate and up in one code layout (MLX rows or ``affine_repack``'s), down in
    either (results are the same bit for bit). The hidden activation is rounded to the
    activation dtype between the two projections, as the reference executor does
    (``metile/backends/mlx_quantized.py:1829-1830``).
    """
    gw, gs, gb = gate
    uw, us, ub = up
    dw, ds, db = down
    if _repacked(gw) != _repacked(uw):
        raise ValueError("affine MLP gate and up weights must share one code layout")
    _require_device(values, gw, gs, gb, uw, us, ub, dw, ds, db, residual)
    code = _dtype_code(values.dtype)
    _check_params(values, gw, gs, gb, group_size, bits, "affine MLP gate")
    _check_params(values, uw, us, ub, group_size, bits, "affine MLP up")
    hdim = values.shape[-1]
    idim = _code_shape(gw, bits)[0]
    if _code_shape(dw, bits) != (hdim, idim):
        raise ValueError("affine MLP received incompatible down-projection parameters")
    if (tuple(ds.shape) != (hdim, idim // group_size) or tuple(db.shape) != tuple(ds.shape)
            or ds.dtype != values.dtype or db.dtype != values.dtype):
        raise ValueError("affine MLP received incompatible down-projection parameters")
    lead = tuple(values.shape[:-1])
    x = values.reshape(-1, hdim).contiguous()
    m = x.shape[0]
    out = torch.empty(*lead, hdim, dtype=values.dtype, device=values.device)
    if m == 0:
        return out
    res = None
    if residual is not None:
        if tuple(residual.shape) != (*lead, hdim) or residual.dtype != values.dtype:
            raise ValueError("residual must match the affine MLP output shape and dtype")
        res = residual.reshape(m, hdim).contiguous()
    tensors = [_as_u32(gw), gs.contiguous(), gb.contiguous(), _as_u32(uw), us.contiguous(),
               ub.contiguous(), _as_u32(dw), ds.contiguous(), db.contiguous()]
    L = _lib.lib()
    need = L.mt_affine_mlp_workspace_bytes(m, hdim, idim, group_size, bits)
    ws = workspace(values.device, need)
    args = (x.data_ptr(), *[t.data_ptr() for t in tensors], _ptr(res), out.data_ptr(), m, hdim,
            idim, group_size, bits, code)
    tail = (ws.data_ptr(), ws.numel(), _stream_handle(values.device))
    if _repacked(gw) == _repacked(dw):
        fn = L.mt_affine_mlp_repacked if _repacked(gw) else L.mt_affine_mlp
        _lib.check(fn(*args, *tail))
    else:
        _lib.check(L.mt_affine_mlp_layouts(*args, _layout_code(gw), _layout_code(dw), *tail))
    return out


class BoundMlp:
    """``affine_mlp`` over fixed weights, for callers that run the same MLP on every token (the
    executors and the model-level caller). The weights are validated and their device pointers
    taken once; a call checks only the activations and the residual, takes a workspace and makes
    the one C-ABI call, which keeps the host cost of an eager decode step near the C ABI's own.
    Results are those of ``affine_mlp`` over the same triples, bit for bit (the same entry
    point). Inputs it does not take (another dtype, width or device) go through ``affine_mlp``,
    which raises the reference's errors."""

    __slots__ = ("triples", "group_size", "bits", "hdim", "idim", "dtype", "device", "code",
                 "wptrs", "layouts", "need", "keep")

    def __init__(self, gate, up, down, *, group_size=64, bits=4):
        gw, gs, gb = gate
        uw, us, ub = up
        dw, ds, db = down
        if _repacked(gw) != _repacked(uw):
            raise ValueError("affine MLP gate and up weights must share one code layout")
        _require_device(gw, gs, gb, uw, us, ub, dw, ds, db)
        self.code = _dtype_code(gs.dtype)
        self.idim, self.hdim = _code_shape(gw, bits)
        probe = torch.empty(1, self.hdim, dtype=gs.dtype, device="meta")
        _check_params(probe, gw, gs, gb, group_size, bits, "affine MLP gate")
        _check_params(probe, uw, us, ub, group_size, bits, "affine MLP up")
        if (_code_shape(dw, bits) != (self.hdim, self.idim)
                or tuple(ds.shape) != (self.hdim, self.idim // group_size)
                or tuple(db.shape) != tuple(ds.shape) or ds.dtype != gs.dtype
                or db.dtype != gs.dtype or us.dtype != gs.dtype or gb.dtype != gs.dtype):
            raise ValueError("affine MLP received incompatible down-projection parameters")
        self.triples = (gate, up, down)
        self.group_size, self.bits = group_size, bits
        self.dtype, self.device = gs.dtype, gs.device
        self.keep = [_as_u32(gw), gs.contiguous(), gb.contiguous(), _as_u32(uw), us.contiguous(),
                     ub.contiguous(), _as_u32(dw), ds.contiguous(), db.contiguous()]
        self.wptrs = tuple(t.data_ptr() for t in self.keep)
        self.layouts = (_layout_code(gw), _layout_code(dw))
        self.need = {}

    def _general(self, values, residual):
        return affine_mlp(values, *self.triples, group_size=self.group_size, bits=self.bits,
                          residual=residual)

    def __call__(self, values, residual=None):
        if (values.dtype != self.dtype or values.device != self.device
                or values.shape[-1] != self.hdim):
            return self._general(values, residual)
        lead = values.shape[:-1]
        x = values.reshape(-1, self.hdim)
        if not x.is_contiguous():
            x = x.contiguous()
        m = x.shape[0]
        out = torch.empty(*lead, self.hdim, dtype=self.dtype, device=self.device)
        if m == 0:
            return out
        rptr = None
        if residual is not None:
            if (residual.shape != out.shape or residual.dtype != self.dtype
                    or residual.device != self.device):
                return self._general(values, residual)
            r = residual.reshape(m, self.hdim)
            if not r.is_contiguous():
                r = r.contiguous()
            rptr = r.data_ptr()
        L = _lib.lib()
        stream = _stream_handle(self.device)
        for attempt in (0, 1):
            need = self.need.get(m) if attempt == 0 else None
            if need is None:  # installed plans may change the need: refreshed on a refusal
                need = self.need[m] = L.mt_affine_mlp_workspace_bytes(
                    m, self.hdim, self.idim, self.group_size, self.bits)
            ws = workspace(self.device, need, stream)
            st = L.mt_affine_mlp_layouts(
                x.data_ptr(), *self.wptrs, rptr, out.data_ptr(), m, self.hdim, self.idim,
                self.group_size, self.bits, self.code, *self.layouts, ws.data_ptr(), ws.numel(),
                stream)
            if st != _lib.MT_ERR_WORKSPACE:
                break
        _lib.check(st)
        return out


def affine_dequantize(weight, scales, biases, *, group_size=64, bits=4):
    """Bit-exact fp32 ``q * s + b`` as a ``[N, K]`` float32 tensor
    (``kernels/affine_qmv.py:41-51``)."""
    if biases is None:
        raise ValueError("dequantize requires biases matching the scales")
    if bits not in (4, 8):
        raise ValueError("dequantize supports 4- and 8-bit codes")
    if weight.ndim != 2 or scales.ndim != 2:
        raise ValueError("expected packed weight and matching two-dimensional parameters")
    n = weight.shape[0]
    k = weight.shape[1] * 32 // bits
    if (group_size < 1 or k % group_size or tuple(scales.shape) != (n, k // group_size)
            or biases.dtype != scales.dtype or tuple(biases.shape) != tuple(scales.shape)):
        raise ValueError("dequantize received incompatible quantization parameters")
    _require_device(weight, scales, biases)
    code = _dtype_code(scales.dtype)
    out = torch.empty(n, k, dtype=torch.float32, device=weight.device)
    w = _as_u32(weight)
    s, b = scales.contiguous(), biases.contiguous()
    _lib.check(_lib.lib().mt_affine_dequantize(
        w.data_ptr(), s.data_ptr(), b.data_ptr(), out.data_ptr(), n, k, group_size, bits, code,
        _stream_handle(weight.device)))
    return out


def affine_repack(weight, *, bits=4):
    """Step-major repack of MLX affine codes for the small-row kernels: the ``8*bits`` bytes
    holding codes ``[64t, 64t + 64)`` of row ``n`` become ``packed[t, n]``, so the codes every
    column of a strip needs for one K step are contiguous. Returns ``[K/64, N, 2*bits]`` words
    of the input's dtype. A one-time cost (one read and one write of the codes); the kernels'
    results over it equal those over the MLX rows bit for bit."""
    _require_device(weight)
    if bits not in (4, 8):
        raise ValueError("affine repack supports 4- and 8-bit codes")
    if weight.ndim != 2:
        raise ValueError("expected packed weight and matching two-dimensional parameters")
    n = weight.shape[0]
    k = weight.shape[1] * 32 // bits
    if n < 1 or k < 64 or k % 64:
        raise ValueError("affine repack requires K to be a positive multiple of 64")
    w = _as_u32(weight)
    out = torch.empty(k // 64, n, 2 * bits, dtype=w.dtype, device=w.device)
    _lib.check(_lib.lib().mt_affine_repack(w.data_ptr(), out.data_ptr(), n, k, bits,
                                           _stream_handle(w.device)))
    return out


def affine_matmul(values, weight, scales, biases, *, group_size=64, bits=4):
    """Prefill ``values @ dequantize(weight).T`` for many rows: codes are dequantized to the
    activation type in LDS and multiplied on the matrix cores (fp32 accumulation), the
    semantics of MLX's quantized matmul for large row counts
    (``metile/backends/mlx_affine.py:142-154``)."""
    if biases is None:
        raise ValueError("affine matmul requires affine quantization biases")
    _require_device(values, weight, scales, biases)
    code = _dtype_code(values.dtype)
    _check_params(values, weight, scales, biases, group_size, bits, "affine matmul")
    k = values.shape[-1]
    n = weight.shape[0]
    lead = tuple(values.shape[:-1])
    x = values.reshape(-1, k).contiguous()
    m = x.shape[0]
    out = torch.empty(*lead, n, dtype=values.dtype, device=values.device)
    if m == 0:
        return out
    w = _as_u32(weight)
    s, b = scales.contiguous(), biases.contiguous()
    lib = _lib.lib()
    need = lib.mt_affine_gemm_workspace_bytes(m, k, n, group_size, bits)
    ws = workspace(values.device, need) if need else None
    _lib.check(lib.mt_affine_gemm(
        x.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(), out.data_ptr(), m, k, n,
        group_size, bits, code, _ptr(ws), 0 if ws is None else ws.numel(),
        _stream_handle(values.device)))
    return out


@dataclass(frozen=True)
class AffineWeight:
    """One affine 4-bit weight for the prefill path, ``shape = (K, N)``.

    Counterpart of ``MLXAffineWeight`` (``metile/backends/mlx_affine.py:66-114``). The gfx950
    GEMM reads the native MLX output-major words directly, so no K-major repack is kept.
    """

    native_weight: torch.Tensor
    native_scales: torch.Tensor
    native_biases: torch.Tensor
    shape: tuple
    group_size: int = 64
    bits: int = 4

    @classmethod
    def from_torch(cls, weight, scales, biases, *, group_size=64, bits=4):
        if group_size != 64 or bits != 4:
            raise ValueError(
                f"affine prefill weights require group size 64 and 4 bits, got {group_size} and "
                f"{bits}")
        if biases is None:
            raise ValueError("native affine QMV requires affine biases")
        if weight.ndim != 2 or scales.ndim != 2 or biases.shape != scales.shape:
            raise ValueError("expected packed weight and matching two-dimensional parameters")
        k = weight.shape[1] * 32 // bits
        return cls(weight, scales, biases, (k, weight.shape[0]), group_size, bits)


# ---------------------------------------------------------------------------------------------
# reference-named entry points (metile/backends/mlx_quantized.py)
# ---------------------------------------------------------------------------------------------


def mlx_affine_qmv(values, weight, scales, biases, *, group_size=64, bits=4, block=32,
                   outputs_per_simdgroup=1, decode_dtype="f32"):
    """Drop-in for ``mlx_affine_qmv`` (``metile/backends/mlx_quantized.py:691-714``).

    ``block``, ``outputs_per_simdgroup`` and ``decode_dtype`` choose among the reference's
    Metal schedules; the gfx950 kernel has one schedule and always decodes exactly in fp32, so
    they are validated and otherwise unused.
    """
    if block not in (32, 64, 128, 256) or outputs_per_simdgroup not in (1, 2, 4, 8):
        raise ValueError("unsupported affine QMV schedule")
    if decode_dtype not in ("f32", "f16"):
        raise ValueError("decode_dtype must be 'f32' or 'f16'")
    return affine_qmv(values, weight, scales, biases, group_size=group_size, bits=bits)


def mlx_affine_residual_qmv(values, weight, scales, biases, residual, *, group_size=64, bits=4,
                            autotune=True):
    """Drop-in for ``mlx_affine_residual_qmv`` with the reference's guards
    (``metile/backends/mlx_quantized.py:1538-1568``). With ``autotune`` the first call of a
    shape takes its tuned plan (``metile_amd.tuning``: cached, else measured once)."""
    mlx_affine_residual_qmv_guards(values, weight, scales, biases, residual,
                                   group_size=group_size, bits=bits)
    if autotune and values.numel():
        _tuning.ensure_qmv_plans(values, (weight, scales, biases), group_size=group_size,
                                 bits=bits)
    return affine_qmv(values, weight, scales, biases, group_size=group_size, bits=bits,
                      residual=residual)


def _swiglu_guards(values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                   up_biases, group_size, bits):
    if not ((bits == 4 and group_size == 64) or (bits == 8 and group_size in {32, 64, 128})):
        raise ValueError("affine SwiGLU requires 4-bit group-64 or 8-bit group-32/64/128 weights")
    if gate_biases is None or up_biases is None:
        raise ValueError("affine SwiGLU requires affine quantization biases")
    if (values.dtype != gate_scales.dtype or values.dtype != gate_biases.dtype
            or gate_weight.shape != up_weight.shape or gate_scales.shape != up_scales.shape
            or gate_biases.shape != up_biases.shape):
        raise ValueError("affine SwiGLU requires matching gate/up weights and parameters")


def mlx_affine_swiglu(values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                      up_biases, *, group_size=64, bits=4, autotune=True):
    """Drop-in for ``mlx_affine_swiglu`` with the reference's guards
    (``metile/backends/mlx_quantized.py:1645-1670``). With ``autotune`` the first call of a
    shape takes its tuned plan (``metile_amd.tuning``: cached, else measured once), as the
    reference's tuned dispatch does (``:1671-1720``)."""
    _swiglu_guards(values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                   up_biases, group_size, bits)
    if autotune and values.numel():
        _tuning.ensure_qmv_plans(values, (gate_weight, gate_scales, gate_biases, up_weight,
                                          up_scales, up_biases), group_size=group_size, bits=bits)
    return affine_swiglu(values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                         up_biases, group_size=group_size, bits=bits)


def mlx_affine_swiglu_dispatches():
    """This process's SwiGLU dispatch decisions (``metile/backends/mlx_quantized.py:1835-1852``):
    one dict per resolved dispatch shape with its plan, layout and source
    (``metile_amd.tuning.dispatches``)."""
    return _tuning.dispatches("swiglu")


def mlx_affine_residual_qmv_dispatches():
    """This process's one-projection (residual) QMV dispatch decisions
    (``metile/backends/mlx_quantized.py:1627-1642``; ``metile_amd.tuning.dispatches``)."""
    return _tuning.dispatches("qmv")


def mlx_affine_swiglu_qmv(values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                          up_biases, *, group_size=64, bits=4, block=32, outputs_per_simdgroup=1,
                          decode_dtype="f32"):
    """Drop-in for the fixed-schedule ``mlx_affine_swiglu_qmv``
    (``metile/backends/mlx_quantized.py:717-751``)."""
    if block not in (32, 64, 128, 256) or outputs_per_simdgroup not in (1, 2, 4, 8):
        raise ValueError("unsupported affine SwiGLU schedule")
    return affine_swiglu(values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                         up_biases, group_size=group_size, bits=bits)


def repack_mlx_affine_weight(weight, scales, biases, *, bits=4):
    """Drop-in for ``repack_mlx_affine_weight`` (``metile/backends/mlx_quantized.py:754-774``)
    with its guards: returns ``(packed, scales, biases)`` for ``mlx_affine_qmv_nax`` and
    ``mlx_affine_swiglu_qmv_nax``. The reference repacks to the K-major nibble layout its NAX
    kernels read (and transposes the scales); here ``packed`` is ``affine_repack``'s step-major
    layout, which these kernels read, and the scales and biases keep their layout."""
    if biases is None:
        raise ValueError("native affine QMV requires affine biases")
    if weight.ndim != 2 or scales.ndim != 2 or biases.shape != scales.shape:
        raise ValueError("expected packed weight and matching two-dimensional parameters")
    return affine_repack(weight, bits=bits), scales, biases


def mlx_affine_qmv_nax(values, packed, scales, biases, *, output_features, group_size=64,
                       bits=4, block=32):
    """Drop-in for ``mlx_affine_qmv_nax`` (``metile/backends/mlx_quantized.py:777-797``): the
    QMV over weights from ``repack_mlx_affine_weight``. ``block`` picks among the reference's
    Metal schedules and is validated only."""
    if block not in (32, 64, 128, 256):
        raise ValueError("unsupported affine QMV schedule")
    if packed.ndim != 3 or packed.shape[1] != output_features:
        raise ValueError("expected repacked weights with output_features columns")
    return affine_qmv(values, packed, scales, biases, group_size=group_size, bits=bits)


def mlx_affine_swiglu_qmv_nax(values, gate_packed, gate_scales, gate_biases, up_packed,
                              up_scales, up_biases, *, output_features, group_size=64, bits=4,
                              block=32):
    """Drop-in for ``mlx_affine_swiglu_qmv_nax`` (``metile/backends/mlx_quantized.py:800-831``):
    the fused gate/up SwiGLU over weights from ``repack_mlx_affine_weight``."""
    if block not in (32, 64, 128, 256):
        raise ValueError("unsupported affine SwiGLU schedule")
    if gate_packed.ndim != 3 or gate_packed.shape[1] != output_features:
        raise ValueError("expected repacked weights with output_features columns")
    return affine_swiglu(values, gate_packed, gate_scales, gate_biases, up_packed, up_scales,
                         up_biases, group_size=group_size, bits=bits)


def _fidelity_gate(result, reference, what):
    """Raise unless ``result`` passes the reference tuner's affine fidelity gate against the
    native composition (``metile/backends/mlx_quantized.py:1256-1272,1297``). The reference
    falls back to the native path on failure; here a failure is an error."""
    from .fidelity import affine_swiglu_compatible

    if result.numel() and not affine_swiglu_compatible(result, reference):
        raise RuntimeError(f"{what}: the gfx950 kernel failed the fidelity gate against the "
                           "native quantized-matmul composition on the sample input")


def mlx_affine_swiglu_executor(sample_values, gate_weight, gate_scales, gate_biases, up_weight,
                               up_scales, up_biases, *, group_size=64, bits=4, autotune=True):
    """Drop-in for ``mlx_affine_swiglu_executor`` (``metile/backends/mlx_quantized.py:1723``):
    validates once, repacks the weights ahead of time (``affine_repack``, as the reference's
    executor does for its repacked schedules, ``metile/backends/mlx_quantized.py:1082-1100``),
    tunes the plan of the sample's shape over both code layouts and keeps the faster
    (``metile_amd.tuning.ensure_qmv_layout``; cached decisions are reused), checks the kernel
    against the native composition on the sample (the reference tuner's fidelity gate) and
    returns ``execute(values)`` bound to the kept weights."""
    from .native import native_affine_swiglu

    _swiglu_guards(sample_values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                   up_biases, group_size, bits)
    mlx = (gate_weight, gate_scales, gate_biases, up_weight, up_scales, up_biases)
    packed = (affine_repack(gate_weight, bits=bits), gate_scales, gate_biases,
              affine_repack(up_weight, bits=bits), up_scales, up_biases)
    kept = packed
    if autotune:
        layout = _tuning.ensure_qmv_layout(sample_values, {"repacked": packed, "mlx": mlx},
                                           group_size=group_size, bits=bits)
        kept = packed if layout == "repacked" else mlx
    del packed
    _fidelity_gate(
        affine_swiglu(sample_values, *kept, group_size=group_size, bits=bits),
        native_affine_swiglu(sample_values, *mlx, group_size=group_size, bits=bits),
        "affine SwiGLU")

    def execute(values):
        return affine_swiglu(values, *kept, group_size=group_size, bits=bits)

    return execute


def mlx_affine_mlp_executor(sample_values, gate_weight, gate_scales, gate_biases, up_weight,
                            up_scales, up_biases, down_weight, down_scales, down_biases,
                            sample_residual, *, group_size=64, bits=4, autotune=True):
    """Drop-in for ``mlx_affine_mlp_executor`` (``metile/backends/mlx_quantized.py:1770-1832``):
    runs every argument check, repacks the three weights ahead of time (``affine_repack``),
    tunes the plans of both stages at the sample's shape (``metile_amd.tuning``), gates the
    SwiGLU stage and, on the sample's hidden activation, the residual stage against
    the native compositions (the reference tuner's fidelity gate), and returns
    ``execute(values, residual) = down(swiglu(values)) + residual`` over the repacked weights
    (one C-ABI call)."""
    # Every argument check first (on a shape-only stand-in for the hidden activation), then
    # the kernels.
    _swiglu_guards(sample_values, gate_weight, gate_scales, gate_biases, up_weight, up_scales,
                   up_biases, group_size, bits)
    probe = torch.empty((*sample_values.shape[:-1], gate_weight.shape[0]),
                        dtype=sample_values.dtype, device="meta")
    mlx_affine_residual_qmv_guards(probe, down_weight, down_scales, down_biases, sample_residual,
                                   group_size=group_size, bits=bits)
    gate = (affine_repack(gate_weight, bits=bits), gate_scales, gate_biases)
    up = (affine_repack(up_weight, bits=bits), up_scales, up_biases)
    down = (affine_repack(down_weight, bits=bits), down_scales, down_biases)
    mlx = ((gate_weight, gate_scales, gate_biases), (up_weight, up_scales, up_biases),
           (down_weight, down_scales, down_biases))
    return bind_mlp_executor(sample_values, mlx, (gate, up, down), sample_residual,
                             group_size=group_size, bits=bits, autotune=autotune)


def bind_mlp_executor(sample_values, mlx, packed, sample_residual, *, group_size=64, bits=4,
                      autotune=True):
    """The steps of ``mlx_affine_mlp_executor`` after its argument checks, for weights already
    repacked: ``mlx`` and ``packed`` are the (gate, up, down) triples in MLX layout and
    repacked. For each row bucket it serves (the sample's first, others on their first call
    outside graph capture) both stages are tuned over both code layouts and each takes the layout
    its plan reads fastest (``metile_amd.tuning.ensure_qmv_layout``; without ``autotune``, the
    repacked codes): at Qwen2.5-1.5B shape, one row keeps both stages in MLX rows (GEMV
    kernel), four rows or more the repacked codes. Both are held (the MLX triples are the
    caller's). The
    sample's results are gated against the native compositions. Returns
    ``execute(values, residual)``."""
    from .native import native_affine_residual_qmv, native_affine_swiglu

    (gate_weight, gate_scales, gate_biases), (up_weight, up_scales, up_biases), \
        (down_weight, down_scales, down_biases) = mlx
    chosen = {}  # row bucket -> (gate, up, down) in the layouts picked for it

    chunk = 16 if group_size == 32 else 32  # rows of one dispatch

    def bucket(values):
        rows = values.numel() // values.shape[-1]
        return _tuning.row_bucket(min(max(rows, 1), chunk))

    def stages(values):
        key = bucket(values)
        if key in chosen:
            return chosen[key]
        gate, up, down = packed
        if not autotune:
            return packed
        if torch.cuda.is_current_stream_capturing():
            return packed  # decided on a later call outside capture
        x = values.reshape(-1, values.shape[-1])
        layout = _tuning.ensure_qmv_layout(
            x, {"repacked": (*gate, *up), "mlx": (*mlx[0], *mlx[1])},
            group_size=group_size, bits=bits)
        if layout == "mlx":
            gate, up = mlx[0], mlx[1]
        hidden = affine_swiglu(x, *gate, *up, group_size=group_size, bits=bits)
        layout = _tuning.ensure_qmv_layout(hidden, {"repacked": down, "mlx": mlx[2]},
                                           group_size=group_size, bits=bits)
        if layout == "mlx":
            down = mlx[2]
        chosen[key] = (gate, up, down)
        return chosen[key]

    gate, up, down = stages(sample_values)
    hidden = affine_swiglu(sample_values, *gate, *up, group_size=group_size, bits=bits)
    _fidelity_gate(
        hidden,
        native_affine_swiglu(sample_values, gate_weight, gate_scales, gate_biases, up_weight,
                             up_scales, up_biases, group_size=group_size, bits=bits),
        "affine SwiGLU")
    _fidelity_gate(
        affine_qmv(hidden, *down, group_size=group_size, bits=bits, residual=sample_residual),
        native_affine_residual_qmv(hidden, down_weight, down_scales, down_biases,
                                   sample_residual, group_size=group_size, bits=bits),
        "affine residual QMV")

    bound = {}  # row bucket -> BoundMlp over the layouts decided for it

    def execute(values, residual):
        key = bucket(values)
        call = bound.get(key)
        if call is None:
            call = BoundMlp(*stages(values), group_size=group_size, bits=bits)
            if key in chosen or not autotune:  # final: decided (or never tuned)
                bound[key] = call
        return call(values, residual)

    return execute


def mlx_affine_residual_qmv_guards(values, weight, scales, biases, residual, *, group_size=64,
                                   bits=4):
    """The argument checks of ``mlx_affine_residual_qmv`` without running it."""
    if group_size != 64 or bits != 4:
        raise ValueError("affine residual QMV requires 4-bit weights with group size 64")
    if biases is None:
        raise ValueError("affine residual QMV requires affine quantization biases")
    k = values.shape[-1]
    n = weight.shape[0]
    shape = (n, k // group_size)
    if (weight.ndim != 2 or weight.shape[1] * 32 // bits != k or tuple(scales.shape) != shape
            or tuple(biases.shape) != shape):
        raise ValueError("affine residual QMV received incompatible quantization parameters")
    if scales.dtype != values.dtype or biases.dtype != values.dtype:
        raise ValueError("affine residual QMV parameters must match the input dtype")
    if tuple(residual.shape) != (*values.shape[:-1], n) or residual.dtype != values.dtype:
        raise ValueError("residual must match the affine QMV output shape and dtype")


def mlx_affine_matmul_dispatches():
    """This process's prefill GEMM dispatch decisions (``metile/backends/mlx_affine.py:409-422``;
    ``metile_amd.tuning.dispatches``)."""
    return _tuning.dispatches("matmul")


def mlx_affine_matmul(values, weight, *, autotune=True):
    """Drop-in for ``mlx_affine_matmul`` (``metile/backends/mlx_affine.py:359-406``) with the
    reference's guards; with ``autotune`` the first call of a shape takes its tuned GEMM plan
    (``metile_amd.tuning``), as the reference's tuned dispatch does (``:380-406``). The reference's Metal path takes float16 only; the gfx950 GEMM also
    takes bfloat16 (BASELINE config 4 is bf16), and any other dtype raises ``TypeError``."""
    if not isinstance(weight, AffineWeight):
        raise TypeError("weight must be an AffineWeight")
    if values.ndim < 2 or values.shape[-1] != weight.shape[0]:
        raise ValueError("expected values[..., K] and a KxN affine weight")
    if values.dtype not in _DTYPES:
        raise TypeError("affine matmul requires float16 or bfloat16 activations")
    if autotune and values.numel() and weight.bits == 4 and weight.group_size >= 64:
        _tuning.ensure_gemm_plan(values, weight.native_weight, weight.native_scales,
                                 weight.native_biases, group_size=weight.group_size)
    return affine_matmul(values, weight.native_weight, weight.native_scales,
                         weight.native_biases, group_size=weight.group_size, bits=weight.bits)
