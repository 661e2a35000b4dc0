"""Patch mechanics of the model-level caller on the CPU (no kernels run): the gated-MLP class
of a tiny Hugging Face model is patched and restored, unsupported modules (plain nn.Linear
projections, host tensors) keep the original forward and its results, and a call with fewer
rows than ``min_rows`` restores the original forward for good, as
``metile/integrations/mlx_lm.py:3898-3928`` does."""

from __future__ import annotations

import pytest
import torch

import metile_amd as mt

transformers = pytest.importorskip("transformers")


def _tiny():
    cfg = transformers.Qwen2Config(hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                                   num_attention_heads=2, num_key_value_heads=1, vocab_size=97,
                                   max_position_embeddings=64)
    torch.manual_seed(0)
    return transformers.Qwen2ForCausalLM(cfg).eval()


def test_patch_and_restore_keep_unsupported_modules_on_the_original_forward():
    model = _tiny()
    mlp_class = type(model.model.layers[0].mlp)
    original = mlp_class.forward
    ids = torch.arange(10).view(1, 10)
    with torch.no_grad():
        want = model(ids).logits
        reps = mt.patch_quantized_mlp(model)
        try:
            assert mlp_class.forward is not original
            assert mlp_class.forward._metile_original is original
            assert mt.patch_quantized_mlp(model) == []  # already patched
            got = model(ids).logits
        finally:
            mt.restore_patches(reps)
    assert mlp_class.forward is original
    torch.testing.assert_close(got, want, rtol=0, atol=0)


def test_fewer_rows_than_min_rows_restores_the_original_forward():
    model = _tiny()
    mlp_class = type(model.model.layers[0].mlp)
    original = mlp_class.forward
    reps = mt.patch_quantized_mlp(model, min_rows=4)
    try:
        with torch.no_grad():
            model(torch.arange(2).view(1, 2))
        assert mlp_class.forward is original
    finally:
        mt.restore_patches(reps)
    assert mlp_class.forward is original


def test_patch_argument_guards():
    model = _tiny()
    with pytest.raises(ValueError, match="minimum rows must be positive"):
        mt.patch_quantized_mlp(model, min_rows=0)
    with pytest.raises(ValueError, match="must not be smaller than its minimum"):
        mt.patch_quantized_mlp(model, min_rows=4, max_rows=2)


def test_quantizer_guards():
    w = torch.zeros(8, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm device"):
        mt.affine_quantize(w)
    with pytest.raises(ValueError, match="compressed down-projection weights must be matrices"):
        mt.CompressedDownWeight.quantize(w[0])
    with pytest.raises(ValueError, match="must be affine8 or mxfp8"):
        mt.CompressedDownWeight.quantize(w, format="int3")


def test_graph_fusion_patches_recognised_blocks_and_falls_back_off_device():
    model = _tiny()
    block_class = type(model.model.layers[0])
    original = block_class.forward
    ids = torch.arange(10).view(1, 10)
    with torch.no_grad():
        want = model(ids).logits
        reps = mt.patch_graph_fusion(model)
        try:
            assert len(reps) == 1 and block_class.forward is not original
            assert block_class.forward._metile_original is original
            assert mt.patch_graph_fusion(model) == []  # already patched
            got = model(ids).logits  # host tensors: every block takes the original forward
        finally:
            mt.restore_patches(reps)
    assert block_class.forward is original
    torch.testing.assert_close(got, want, rtol=0, atol=0)


def test_graph_fusion_leaves_unrecognised_blocks_alone():
    model = _tiny()
    layer_class = type(model.model.layers[0])

    class CustomLayer(layer_class):  # same structure, not a registered class
        pass

    for layer in model.model.layers:
        layer.__class__ = CustomLayer
    assert mt.patch_graph_fusion(model) == []
    with pytest.raises(ValueError, match="minimum rows must be positive"):
        mt.patch_graph_fusion(model, quantized_mlp_min_rows=0)
