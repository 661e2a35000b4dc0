"""The quantizer and the model-level caller on the GPU.

* ``affine_quantize`` (``mt_affine_quantize``) equals the oracle's restatement bit for bit.
* ``CompressedDownWeight`` (the reference's INT8 down-projection weight) quantizes and projects
  within the kernel tolerance of the oracle.
* Token equality, after the reference's ``tests/test_model_equivalence.py``: tiny Qwen2 and
  Llama models (random weights from a seeded config; no checkpoints are available offline)
  have their MLP projections quantized, then decode greedily once with the original gated-MLP
  forward (three projections, the activation in torch) and once patched: to the fused SwiGLU
  kernel (``patch_quantized_mlp``), or to one MLP executor call per layer with the residual
  add in the down projection (``patch_graph_fusion``); unquantized bf16 models patched by
  ``patch_graph_fusion`` run the dense SwiGLU and residual kernels at one row. The two differ only in where SwiGLU rounds, so the logits agree to a few bf16 units
  in the last place and the tokens must agree; a divergence is allowed only at a step where
  the measured logit difference is large enough to reorder the two tokens involved.
  Attention runs in float32 (bf16 batched products with transposed operands are kept off the
  GPU here).
"""

from __future__ import annotations


import numpy as np
import pytest
import torch

import metile_amd as mt
from oracle import affine as O
from tests.helpers import act_to_torch, torch_to_act

pytestmark = pytest.mark.gpu

# Largest logit difference allowed between the original and the patched run, as a fraction of
# the largest logit magnitude: four bf16 units in the last place (2^-8 each) of the largest.
LOGIT_TOLERANCE = 4 * 2.0 ** -8


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)


@pytest.mark.parametrize("bits,g,dtype,n,k", [(4, 64, "bf16", 96, 512), (8, 32, "bf16", 64, 256),
                                              (4, 128, "f16", 40, 1024), (8, 64, "f16", 8960, 256),
                                              (4, 64, "bf16", 1536, 8960)])
def test_quantize_is_the_oracle(bits, g, dtype, n, k):
    rng = np.random.default_rng(n * 7 + k + bits)
    dense = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    dense[0, :g] = 0.0                      # a zero group
    dense[1, :g] = 0.375                    # a constant group
    dense[2, :g] = np.linspace(-1, 1, g)    # |min| == |max|
    w = O.from_f32(dense, dtype)
    w_q, s, b = mt.affine_quantize(act_to_torch(w, dtype), group_size=g, bits=bits)
    torch.cuda.synchronize()
    ow, os_, ob = O.affine_quantize(w, g, bits, dtype)
    np.testing.assert_array_equal(w_q.cpu().numpy().view(np.uint32), ow)
    np.testing.assert_array_equal(torch_to_act(s, dtype), os_)
    np.testing.assert_array_equal(torch_to_act(b, dtype), ob)


def test_compressed_down_weight_projects_like_the_oracle():
    rng = np.random.default_rng(5)
    dense = O.from_f32((rng.standard_normal((1536, 1024)) * 0.02).astype(np.float32), "bf16")
    cw = mt.CompressedDownWeight.quantize(act_to_torch(dense, "bf16"), group_size=64)
    assert cw.format == "affine8" and cw.shape == (1536, 1024)
    x = O.make_activations(3, 1024, 5)
    y = torch_to_act(cw(act_to_torch(x, "bf16")), "bf16")
    w_q = cw.values.cpu().numpy().view(np.uint32)
    ref = O.affine_qmv(x, w_q, torch_to_act(cw.scales, "bf16"), torch_to_act(cw.biases, "bf16"),
                       64, 8)
    assert O.tolerance_error(y, ref) <= 2e-3
    with pytest.raises(ValueError, match="group size"):
        mt.CompressedDownWeight.quantize(act_to_torch(dense, "bf16"), group_size=16)


def _fp32_attention(module, query, key, value, attention_mask, **kwargs):
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    mask = attention_mask
    if mask is not None and mask.is_floating_point():
        mask = mask.float()
    out, weights = sdpa_attention_forward(module, query.float(), key.float(), value.float(), mask,
                                          **kwargs)
    return out.to(query.dtype), weights


def _tiny_model(family, quantize=True):
    transformers = pytest.importorskip("transformers")
    transformers.AttentionInterface.register("metile_fp32_sdpa", _fp32_attention)
    common = dict(hidden_size=256, intermediate_size=768, num_hidden_layers=3,
                  num_attention_heads=4, num_key_value_heads=2, vocab_size=1024,
                  max_position_embeddings=256, hidden_act="silu", tie_word_embeddings=False)
    torch.manual_seed(1234)
    if family == "qwen2":
        cfg = transformers.Qwen2Config(**common)
        model = transformers.Qwen2ForCausalLM(cfg)
    else:
        cfg = transformers.LlamaConfig(**common)
        model = transformers.LlamaForCausalLM(cfg)
    model.config._attn_implementation = "metile_fp32_sdpa"
    model = model.to(device="cuda", dtype=torch.bfloat16).eval()
    if quantize:
        assert mt.quantize_mlp(model) == 3
    return model


@torch.no_grad()
def _greedy(model, prompt, steps):
    out = model(prompt, use_cache=True)
    past, logits = out.past_key_values, [out.logits[0, -1].float()]
    tokens = []
    for _ in range(steps):
        nxt = logits[-1].argmax()
        tokens.append(int(nxt))
        out = model(nxt.view(1, 1), past_key_values=past, use_cache=True)
        past = out.past_key_values
        logits.append(out.logits[0, -1].float())
    return tokens, logits


def _decode_patched(model, patch, counted, steps=24):
    """Greedy decode unpatched, then with ``patch(model)`` applied while the module-level
    function ``counted`` of ``metile_amd.model`` counts its calls (with a residual or not)."""
    prompt = torch.randint(0, 1024, (1, 12), generator=torch.Generator().manual_seed(7)).cuda()
    base = _greedy(model, prompt, steps)
    calls = {"plain": 0, "residual": 0}
    original = getattr(mt.model, counted)

    def counting(module, values, *rest):
        calls["residual" if rest and rest[0] is not None else "plain"] += 1
        return original(module, values, *rest)

    setattr(mt.model, counted, counting)
    replacements = patch(model)
    try:
        patched = _greedy(model, prompt, steps)
    finally:
        mt.restore_patches(replacements)
        setattr(mt.model, counted, original)
    assert len(replacements) == 1
    return base, patched, calls


def _assert_same_decode(family, base, patched):
    (base_tokens, base_logits), (tokens, logits) = base, patched
    scale = max(float(l.abs().max()) for l in base_logits)
    worst = 0.0
    for step, (a, b) in enumerate(zip(base_tokens, tokens)):
        diff = float((logits[step] - base_logits[step]).abs().max())
        worst = max(worst, diff / scale)
        # bf16 logits: the two runs differ by a few units in the last place of the largest.
        assert diff <= LOGIT_TOLERANCE * scale, (family, step, diff, scale)
        if a != b:
            # Greedy decoding may only flip where the runs' perturbation can reorder the two.
            margin = float(base_logits[step][a] - base_logits[step][b])
            assert margin <= 2 * diff, (family, step, margin, diff)
            break
    print(f"[{family}] tokens equal: {base_tokens == tokens}, worst logit difference "
          f"{worst:.4f} of the logit scale", flush=True)


@pytest.mark.parametrize("family", ["qwen2", "llama"])
def test_patched_mlp_decodes_the_same_tokens(family):
    model = _tiny_model(family)
    base, patched, calls = _decode_patched(model, mt.patch_quantized_mlp, "_execute_quantized_mlp")
    assert calls == {"plain": 3 * 25, "residual": 0}  # every layer, prompt and 24 steps
    _assert_same_decode(family, base, patched)


@pytest.mark.parametrize("family", ["qwen2", "llama"])
def test_graph_fusion_runs_the_mlp_executor_with_the_residual(family):
    model = _tiny_model(family)
    base, patched, calls = _decode_patched(model, mt.patch_graph_fusion, "_execute_quantized_mlp")
    # every layer of the prompt and of each step: one executor call, residual fused
    assert calls == {"plain": 0, "residual": 3 * 25}
    assert len(mt.model._quantized_mlp_executor_cache) >= 3
    _assert_same_decode(family, base, patched)


@pytest.mark.parametrize("family", ["qwen2", "llama"])
def test_graph_fusion_runs_dense_mlps_at_one_row(family):
    model = _tiny_model(family, quantize=False)
    base, patched, calls = _decode_patched(model, mt.patch_graph_fusion, "_execute_dense_mlp")
    assert calls == {"plain": 0, "residual": 3 * 24}  # decode steps only (one row each)
    _assert_same_decode(family, base, patched)


def test_prefill_rows_take_the_gemm_and_match_the_decode_path():
    model = _tiny_model("qwen2")
    prompt = torch.randint(0, 1024, (1, 140), generator=torch.Generator().manual_seed(9)).cuda()
    with torch.no_grad():
        base = model(prompt).logits[0].float()
        replacements = mt.patch_quantized_mlp(model)
        try:
            fused = model(prompt).logits[0].float()
        finally:
            mt.restore_patches(replacements)
    scale = float(base.abs().max())
    assert float((fused - base).abs().max()) <= LOGIT_TOLERANCE * scale


def test_tuned_graph_fusion_decodes_the_same_tokens(monkeypatch, tmp_path):
    # with the tuner on, the MLP executors pick plans and code layouts per row bucket (the
    # prompt's 12 rows, then one row per decode step); the tokens must still match
    monkeypatch.setenv("METILE_AMD_CACHE_DIR", str(tmp_path))
    monkeypatch.delenv("METILE_AMD_DISABLE_TUNING", raising=False)
    from metile_amd import tuning

    tuning.clear_plans()
    try:
        model = _tiny_model("qwen2")
        base, patched, calls = _decode_patched(model, mt.patch_graph_fusion,
                                               "_execute_quantized_mlp")
        assert calls == {"plain": 0, "residual": 3 * 25}
        decisions = tuning.load_decisions().values()
        assert {(d["rows"], d["nproj"]) for d in decisions} >= {(1, 1), (1, 2), (16, 1), (16, 2)}
        _assert_same_decode("qwen2 tuned", base, patched)
    finally:
        tuning.clear_plans()
