"""Model-level caller: gated MLPs of torch (Hugging Face transformers) models on the gfx950
kernels.

Counterpart of the reference's MLX-LM integration for quantized MLPs
(``metile/integrations/mlx_lm.py:3805-3929``):

* ``QuantizedLinear`` holds one affine-quantized projection, the torch analogue of MLX's
  ``nn.QuantizedLinear``: the MLX-format codes (for the prefill GEMM) and the same codes
  repacked step-major (for the small-row kernels), scales and biases. ``quantize_mlp`` swaps
  the gate/up/down ``nn.Linear`` layers of a model's gated MLPs for them, as quantizing a
  model for MLX-LM does.
* ``patch_quantized_mlp`` replaces the ``forward`` of every gated MLP class in the model, like
  ``_patch_quantized_mlp``: a module whose gate and up projections are supported
  (``_supports_quantized_mlp``: 4-bit, group 64, affine, no bias, SiLU gate, 16-bit
  activations) runs the fused gate/up SwiGLU kernel on its tuned plan and then its down
  projection (``_execute_quantized_mlp``); any other module, or a call with more rows than
  ``max_rows``, runs the original ``forward``; a call with fewer rows than ``min_rows``
  restores the original ``forward`` of that class for good, as the reference does.
* ``patch_graph_fusion`` replaces the ``forward`` of recognised decoder-layer classes, like the
  reference's ``_patch_graph_fusion`` (``metile/integrations/mlx_lm.py:3663-3790``): the
  layer's second residual add moves into the MLP's last kernel. A supported quantized MLP runs
  as one MLP executor call, ``down(swiglu(x)) + residual`` (``_execute_quantized_mlp`` with a
  residual: an executor per module, tuned and gated on first use and cached); a supported
  dense 16-bit MLP at one row runs the dense SwiGLU and residual kernels
  (``_execute_dense_mlp``); anything else runs the original ``forward``. The fused
  residual-RMSNorm part of the reference's pass is outside this build (norm kernels are not on
  the quantized-projection path): the layer norms run as the model defines them.
* ``restore_patches`` undoes the patches.
"""

from __future__ import annotations

import inspect
import weakref

import torch
from torch import nn

from . import tuning as _tuning
from .dense import DenseWeight, mlx_dense_residual_qmv, mlx_dense_swiglu
from .quantize import affine_quantize
from .quantized import affine_matmul, affine_qmv, affine_repack, affine_swiglu, bind_mlp_executor

# Rows at or above which a 4-bit group-64 projection takes the prefill GEMM.
PREFILL_ROWS = 128


class QuantizedLinear(nn.Module):
    """``y = x @ dequantize(W).T`` for an affine-quantized ``[out, in]`` weight, no bias."""

    def __init__(self, weight, scales, biases, *, group_size=64, bits=4):
        super().__init__()
        if weight.ndim != 2 or scales.shape != biases.shape:
            raise ValueError("expected packed weight and matching two-dimensional parameters")
        self.group_size = group_size
        self.bits = bits
        self.mode = "affine"
        self.in_features = weight.shape[1] * 32 // bits
        self.out_features = weight.shape[0]
        self.register_buffer("weight", weight)
        self.register_buffer("packed", affine_repack(weight, bits=bits))
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)

    @classmethod
    def from_linear(cls, linear: nn.Linear, *, group_size=64, bits=4):
        if linear.bias is not None:
            raise ValueError("quantized projections here carry no bias")
        w = linear.weight.detach()
        if w.dtype not in (torch.bfloat16, torch.float16):
            w = w.to(torch.bfloat16)
        return cls(*affine_quantize(w, group_size=group_size, bits=bits),
                   group_size=group_size, bits=bits)

    def forward(self, x):
        rows = x.numel() // x.shape[-1]
        if rows >= PREFILL_ROWS and self.bits == 4 and self.group_size >= 64:
            return affine_matmul(x, self.weight, self.scales, self.biases,
                                 group_size=self.group_size, bits=self.bits)
        return affine_qmv(x, self.packed, self.scales, self.biases,
                          group_size=self.group_size, bits=self.bits)

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"group_size={self.group_size}, bits={self.bits}")


def _model_layers(model):
    """Decoder layers of a causal LM (``model.model.layers``) or of a bare decoder."""
    inner = getattr(model, "model", model)
    return list(getattr(inner, "layers", ()))


def _is_gated_mlp(module) -> bool:
    return all(isinstance(getattr(module, name, None), nn.Module)
               for name in ("gate_proj", "up_proj", "down_proj"))


def _is_silu(act) -> bool:
    if isinstance(act, nn.SiLU):
        return True
    name = type(act).__name__.lower()
    return "silu" in name or "swish" in name


def quantize_mlp(model, *, group_size=64, bits=4):
    """Replace the gate/up/down ``nn.Linear`` projections of every decoder layer's gated MLP
    with ``QuantizedLinear`` (weights quantized on the GPU by ``affine_quantize``). Returns
    the number of MLPs converted."""
    converted = 0
    for layer in _model_layers(model):
        mlp = getattr(layer, "mlp", None)
        if mlp is None or not _is_gated_mlp(mlp):
            continue
        for name in ("gate_proj", "up_proj", "down_proj"):
            lin = getattr(mlp, name)
            if isinstance(lin, nn.Linear):
                setattr(mlp, name, QuantizedLinear.from_linear(lin, group_size=group_size,
                                                               bits=bits))
        converted += 1
    return converted


def _supports_quantized_mlp(module, values) -> bool:
    """The reference's support check (``metile/integrations/mlx_lm.py:3805-3818``); its
    float16-only activation rule is widened to the two 16-bit types these kernels take."""
    gate = getattr(module, "gate_proj", None)
    up = getattr(module, "up_proj", None)
    return (isinstance(gate, QuantizedLinear) and isinstance(up, QuantizedLinear)
            and gate.mode == up.mode == "affine"
            and gate.group_size == up.group_size == 64
            and gate.bits == up.bits == 4
            and _is_silu(getattr(module, "act_fn", None))
            and values.dtype in (torch.float16, torch.bfloat16)
            and values.dtype == gate.scales.dtype
            and values.is_cuda)


def _supports_quantized_residual_mlp(module, values, residual) -> bool:
    """``_supports_quantized_mlp`` plus a supported down projection and a residual of the
    output's shape and dtype (``metile/integrations/mlx_lm.py:3822-3834``)."""
    down = getattr(module, "down_proj", None)
    return (_supports_quantized_mlp(module, values)
            and isinstance(down, QuantizedLinear)
            and down.mode == "affine" and down.group_size == 64 and down.bits == 4
            and tuple(residual.shape) == (*values.shape[:-1], down.out_features)
            and residual.dtype == values.dtype)


# id(module) -> (weak reference to the module, bound executor)
_quantized_mlp_executor_cache: dict[int, tuple] = {}


def _execute_quantized_mlp(module, values, residual=None):
    """``down(swiglu(values)) (+ residual)`` through an MLP executor bound to this module's
    weights in both code layouts: created (tuned per row bucket, fidelity-gated) on first use and
    cached while the module lives (``metile/integrations/mlx_lm.py:3837-3886``); each call is one
    C-ABI call over pre-validated weights (``BoundMlp``). Without a residual this is the
    reference's tuned SwiGLU followed by the module's down projection: the hidden activation is
    rounded to the activation type between the two, as there. Prefill-sized calls (at least
    ``PREFILL_ROWS`` rows), and modules whose down projection is not an affine
    ``QuantizedLinear`` of the same format, run the SwiGLU kernel and then the module's down
    projection (the prefill GEMM at those rows)."""
    gate, up, down = module.gate_proj, module.up_proj, module.down_proj
    rows = values.numel() // values.shape[-1]
    down_ok = (isinstance(down, QuantizedLinear) and down.mode == "affine"
               and down.group_size == gate.group_size and down.bits == gate.bits)
    if residual is None and (rows >= PREFILL_ROWS or not down_ok):
        layouts = {"repacked": (gate.packed, gate.scales, gate.biases,
                                up.packed, up.scales, up.biases),
                   "mlx": (gate.weight, gate.scales, gate.biases,
                           up.weight, up.scales, up.biases)}
        layout = _tuning.ensure_qmv_layout(values, layouts, group_size=gate.group_size,
                                           bits=gate.bits)
        hidden = affine_swiglu(values, *layouts[layout], group_size=gate.group_size,
                               bits=gate.bits)
        return module.down_proj(hidden)
    key = id(module)
    cached = _quantized_mlp_executor_cache.get(key)
    if cached is None or cached[0]() is not module:
        executor = bind_mlp_executor(
            values,
            ((gate.weight, gate.scales, gate.biases), (up.weight, up.scales, up.biases),
             (down.weight, down.scales, down.biases)),
            ((gate.packed, gate.scales, gate.biases), (up.packed, up.scales, up.biases),
             (down.packed, down.scales, down.biases)),
            residual, group_size=gate.group_size, bits=gate.bits)

        def discard(reference, key=key):
            if _quantized_mlp_executor_cache.get(key, (None,))[0] is reference:
                del _quantized_mlp_executor_cache[key]

        cached = (weakref.ref(module, discard), executor)
        _quantized_mlp_executor_cache[key] = cached
    return cached[1](values, residual)


# id(module) -> (weak reference to the module, (gate, up, down) DenseWeight)
_dense_weight_cache: dict[int, tuple] = {}


def _dense_weights(module):
    key = id(module)
    cached = _dense_weight_cache.get(key)
    if cached is None or cached[0]() is not module:
        weights = tuple(DenseWeight.from_torch(getattr(module, name).weight.detach())
                        for name in ("gate_proj", "up_proj", "down_proj"))

        def discard(reference, key=key):
            if _dense_weight_cache.get(key, (None,))[0] is reference:
                del _dense_weight_cache[key]

        cached = (weakref.ref(module, discard), weights)
        _dense_weight_cache[key] = cached
    return cached[1]


def _supports_dense_residual_mlp(module, values, residual) -> bool:
    """A dense gated MLP (three bias-free 16-bit ``nn.Linear`` on the device, SiLU) at one row
    (``metile/integrations/mlx_lm.py:3625-3637``)."""
    lins = [getattr(module, name, None) for name in ("gate_proj", "up_proj", "down_proj")]
    if not all(isinstance(lin, nn.Linear) and lin.bias is None for lin in lins):
        return False
    gate, _, down = lins
    k, n = gate.in_features, gate.out_features
    return (values.numel() // values.shape[-1] == 1
            and _is_silu(getattr(module, "act_fn", None))
            and values.is_cuda and values.dtype in (torch.float16, torch.bfloat16)
            and all(lin.weight.dtype == values.dtype and lin.weight.is_cuda for lin in lins)
            and values.shape[-1] == k and down.in_features == n
            and k % 64 == 0 and n % 64 == 0 and down.out_features % 32 == 0
            and tuple(residual.shape) == (*values.shape[:-1], down.out_features)
            and residual.dtype == values.dtype)


def _execute_dense_mlp(module, values, residual):
    """Dense SwiGLU, then the down projection with the residual in its epilogue
    (``metile/integrations/mlx_lm.py:3657-3660``)."""
    gate, up, down = _dense_weights(module)
    return mlx_dense_residual_qmv(mlx_dense_swiglu(values, gate, up), down.native_weight, residual)


def patch_quantized_mlp(model, *, min_rows=1, max_rows=None):
    """Patch the ``forward`` of every gated MLP class used by ``model``'s decoder layers
    (``metile/integrations/mlx_lm.py:3889-3928``). Returns the list of replacements for
    ``restore_patches``."""
    if min_rows < 1:
        raise ValueError("quantized MLP minimum rows must be positive")
    if max_rows is not None and max_rows < min_rows:
        raise ValueError("quantized MLP maximum rows must not be smaller than its minimum")
    classes = [type(layer.mlp) for layer in _model_layers(model)
               if hasattr(layer, "mlp") and _is_gated_mlp(layer.mlp)]
    replacements = []
    for mlp_class in dict.fromkeys(classes):
        original = mlp_class.forward
        if getattr(original, "_metile_original", None) is not None:
            continue

        def make_replacement(original_forward, cls=mlp_class):
            def forward(self, values):
                rows = values.numel() // values.shape[-1]
                if rows < min_rows:
                    cls.forward = original_forward
                    return original_forward(self, values)
                if max_rows is not None and rows > max_rows:
                    return original_forward(self, values)
                if not _supports_quantized_mlp(self, values):
                    return original_forward(self, values)
                return _execute_quantized_mlp(self, values)

            return forward

        patched = make_replacement(original)
        patched._metile_original = original
        replacements.append((mlp_class, "forward", original))
        mlp_class.forward = patched
    return replacements


# Decoder layers whose forward is the pre-norm block this pass reproduces:
# r = self_attn(input_layernorm(x)); h = x + r; out = h + mlp(post_attention_layernorm(h)).
# Each is also checked for that forward's parameters before it is patched, so a transformers
# release that changes the block is left alone.
_FUSED_BLOCK_CLASSES = frozenset({
    ("transformers.models.llama.modeling_llama", "LlamaDecoderLayer"),
    ("transformers.models.qwen2.modeling_qwen2", "Qwen2DecoderLayer"),
    ("transformers.models.qwen3.modeling_qwen3", "Qwen3DecoderLayer"),
    ("transformers.models.mistral.modeling_mistral", "MistralDecoderLayer"),
})
_BLOCK_PARAMETERS = ("self", "hidden_states", "attention_mask", "position_ids", "past_key_values",
                     "use_cache", "position_embeddings", "kwargs")
_BLOCK_PARTS = ("input_layernorm", "self_attn", "post_attention_layernorm", "mlp")


def _recognised_block(block_class) -> bool:
    if (block_class.__module__, block_class.__name__) not in _FUSED_BLOCK_CLASSES:
        return False
    try:
        names = tuple(inspect.signature(block_class.forward).parameters)
    except (TypeError, ValueError):
        return False
    return names == _BLOCK_PARAMETERS


def patch_graph_fusion(model, *, quantized_mlp_min_rows=1, quantized_mlp_max_rows=None,
                       dense_mlp=True):
    """Fuse each recognised decoder layer's MLP residual add into the MLP's last kernel
    (``metile/integrations/mlx_lm.py:3663-3790``). Returns the replacements for
    ``restore_patches``."""
    if quantized_mlp_min_rows < 1:
        raise ValueError("quantized MLP minimum rows must be positive")
    if quantized_mlp_max_rows is not None and quantized_mlp_max_rows < quantized_mlp_min_rows:
        raise ValueError("quantized MLP maximum rows must not be smaller than its minimum")
    replacements = []
    for block_class in dict.fromkeys(type(layer) for layer in _model_layers(model)):
        if not _recognised_block(block_class):
            continue
        original = block_class.forward
        if getattr(original, "_metile_original", None) is not None:
            continue

        def make_replacement(original_forward):
            def forward(self, hidden_states, attention_mask=None, position_ids=None,
                        past_key_values=None, use_cache=False, position_embeddings=None,
                        **kwargs):
                mlp = getattr(self, "mlp", None)
                rows = hidden_states.numel() // hidden_states.shape[-1]
                quantized = (mlp is not None and all(hasattr(self, p) for p in _BLOCK_PARTS)
                             and rows >= quantized_mlp_min_rows
                             and (quantized_mlp_max_rows is None
                                  or rows <= quantized_mlp_max_rows)
                             and _supports_quantized_residual_mlp(mlp, hidden_states,
                                                                  hidden_states))
                dense = (not quantized and dense_mlp and mlp is not None
                         and all(hasattr(self, p) for p in _BLOCK_PARTS)
                         and _supports_dense_residual_mlp(mlp, hidden_states, hidden_states))
                if not (quantized or dense):
                    return original_forward(self, hidden_states, attention_mask=attention_mask,
                                            position_ids=position_ids,
                                            past_key_values=past_key_values,
                                            use_cache=use_cache,
                                            position_embeddings=position_embeddings, **kwargs)
                attention, _ = self.self_attn(
                    hidden_states=self.input_layernorm(hidden_states),
                    attention_mask=attention_mask, position_ids=position_ids,
                    past_key_values=past_key_values, use_cache=use_cache,
                    position_embeddings=position_embeddings, **kwargs)
                hidden = hidden_states + attention
                normalized = self.post_attention_layernorm(hidden)
                if quantized:
                    return _execute_quantized_mlp(mlp, normalized, hidden)
                return _execute_dense_mlp(mlp, normalized, hidden)

            return forward

        patched = make_replacement(original)
        patched._metile_original = original
        replacements.append((block_class, "forward", original))
        block_class.forward = patched
    return replacements


def restore_patches(replacements):
    """Undo ``patch_quantized_mlp``."""
    for cls, name, original in reversed(replacements):
        setattr(cls, name, original)
