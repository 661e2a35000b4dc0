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
  activations) runs the fused gate/up SwiGLU kernel and then its down projection
  (``_execute_quantized_mlp``); any other module, or a call with more rows than ``max_rows``,
  runs the original ``forward``; a call with fewer rows than ``min_rows`` restores the
  original ``forward`` of that class for good, as the reference does. ``restore_patches``
  undoes the patches.
"""

from __future__ import annotations

import torch
from torch import nn

from .quantize import affine_quantize
from .quantized import affine_matmul, affine_qmv, affine_repack, affine_swiglu

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


def _execute_quantized_mlp(module, values):
    """The fused gate/up SwiGLU kernel, then the module's down projection
    (``metile/integrations/mlx_lm.py:3837-3852``)."""
    gate, up = module.gate_proj, module.up_proj
    hidden = affine_swiglu(values, gate.packed, gate.scales, gate.biases, up.packed, up.scales,
                           up.biases, group_size=gate.group_size, bits=gate.bits)
    return module.down_proj(hidden)


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


def restore_patches(replacements):
    """Undo ``patch_quantized_mlp``."""
    for cls, name, original in reversed(replacements):
        setattr(cls, name, original)
