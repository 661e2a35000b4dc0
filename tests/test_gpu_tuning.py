"""Plans and the tuner on the GPU, through the C ABI.

* Every plan the library lists for a shape (``mt_affine_qmv_plan_candidates``) computes the
  oracle's result within the kernels' tolerance, and under each installed plan the kernels over
  MLX codes and over repacked codes agree bit for bit. The tuner may install any of these plans,
  so all of them are checked, at BASELINE shapes and others (Qwen2.5-0.5B, 8-bit, groups of 32).
* The same for the prefill GEMM's plans, against the native composition.
* The tuner end to end: it measures, installs and persists a decision; a fresh process state
  reads the decision back from the cache without measuring; results under tuned plans stay
  within the tolerance of the oracle.
"""

from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

import metile_amd as mt
from metile_amd import tuning
from oracle import affine as O
from tests.helpers import act_to_torch, affine_to_torch, torch_to_act

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)


@pytest.fixture(autouse=True)
def _clean_plans():
    tuning.clear_plans()
    yield
    tuning.clear_plans()


def _check(name, y, ref, min_exact=0.98):
    err = O.tolerance_error(y, ref, "bf16")
    exact = np.mean(O.to_f32(y, "bf16") == O.to_f32(O.from_f32(ref.astype(np.float32), "bf16"),
                                                     "bf16"))
    assert err <= TOL and exact >= min_exact, (name, err, exact)
    return err


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


# Every (rows, shape, projections) bench.py times is here, so that every plan the tuner may
# install for a timed dispatch has been checked against the oracle: the config-1 MLP stages
# (gate/up 1536 -> 8960 fused, down 8960 -> 1536 with the residual) and config 0
# (1536 -> 8960, one projection) at 1, 2, 4, 8, 16 and 32 rows, config 3 (8 bits,
# 5120 -> 17408) at 1, 8 and 16 rows; then other shapes (Qwen2.5-0.5B, 8 bits, groups of 32).
QMV_SHAPES = (
    [(m, 1536, 8960, 64, 4, 2, False) for m in (1, 2, 4, 8, 16, 32)]
    + [(m, 8960, 1536, 64, 4, 1, True) for m in (1, 2, 4, 8, 16, 32)]
    + [(m, 1536, 8960, 64, 4, 1, False) for m in (1, 2, 4, 8, 16, 32)]
    + [(m, 5120, 17408, 64, 8, 1, False) for m in (1, 8, 16)]
    + [
        (5, 896, 4864, 64, 4, 2, False),
        (3, 4864, 896, 64, 4, 1, True),
        (3, 1024, 1536, 32, 8, 2, False),
        (1, 5120, 2048, 64, 8, 1, False),
        # Llama-3-8B's MLP at one row: 448 strips of gate/up, 224-step down projection
        (1, 4096, 14336, 64, 4, 2, False),
        (1, 14336, 4096, 64, 4, 1, True),
    ]
)


@functools.lru_cache(maxsize=2)
def _oracle_case(k, n, g, bits, nproj, residual, rows):
    """Inputs and the oracle's result at ``rows`` rows (row r of the inputs is the same for
    every row count: the generators fill rows in order)."""
    weights = [O.make_affine_weight(n, k, bits, g, 7, 10 + 2 * p) for p in range(nproj)]
    x = O.make_activations(rows, k, 7)
    res = O.make_activations(rows, n, 7, tensor_id=3) if residual else None
    if nproj == 2:
        ref = O.affine_swiglu(x, weights[0], weights[1], g, bits)
    else:
        ref = O.affine_qmv(x, *weights[0], g, bits, residual=res)
    return weights, x, res, ref


@pytest.mark.parametrize("shape", QMV_SHAPES, ids=lambda s: "x".join(map(str, s[:6])))
def test_every_candidate_plan_matches_the_oracle(shape):
    rows, k, n, g, bits, nproj, residual = shape
    most = max(s[0] for s in QMV_SHAPES if s[1:] == shape[1:])
    weights, x, res, ref = _oracle_case(k, n, g, bits, nproj, residual, most)
    x, ref = x[:rows], ref[:rows]
    res = None if res is None else res[:rows]
    xt = act_to_torch(x, "bf16")
    rt = None if res is None else act_to_torch(res, "bf16")
    mlx = [affine_to_torch(w, "bf16") for w in weights]
    packed = [(mt.affine_repack(w, bits=bits), s, b) for (w, s, b) in mlx]

    def run(ts):
        if nproj == 2:
            return mt.affine_swiglu(xt, *ts[0], *ts[1], group_size=g, bits=bits)
        return mt.affine_qmv(xt, *ts[0], group_size=g, bits=bits, residual=rt)

    cands = tuning.qmv_plan_candidates(rows, k, n, g, bits, nproj)
    assert cands
    worst = 0.0
    for plan in cands:
        print(f"[{shape}] plan {plan}", flush=True)
        tuning.install_qmv_plan(rows, k, n, g, bits, nproj, torch.bfloat16, plan)
        assert tuning.qmv_plan(rows, k, n, g, bits, nproj, torch.bfloat16) == plan
        a, b = run(mlx), run(packed)
        torch.cuda.synchronize()
        assert _same(a, b), plan
        worst = max(worst, _check(str(plan), torch_to_act(a, "bf16"), ref))
    print(f"[{shape}] {len(cands)} plans, worst tolerance_error {worst:.2e}", flush=True)


# The prefill GEMM's plans are held to the contract where the tuner installs them: config 4's
# two projections at M = 512 (every plan the library lists, the planner's included), and two
# ragged shapes. Each must be within tolerance_error 2e-3 of the fp32-accumulated oracle over
# the exact dequantized weights and equal its correctly rounded value in >= 98% of outputs.
GEMM_SHAPES = [(512, 1536, 8960), (512, 8960, 1536), (200, 1024, 1536), (130, 1536, 896)]


@functools.lru_cache(maxsize=1)
def _gemm_case(m, k, n):
    w = O.make_affine_weight(n, k, 4, 64, 8, 10)
    x = O.make_activations(m, k, 8)
    ref = (O.to_f32(x, "bf16") @ O.dequantize(*w, 64, 4, "bf16").T).astype(np.float64)
    return w, x, ref


@pytest.mark.parametrize("m,k,n", GEMM_SHAPES, ids=lambda v: str(v))
def test_every_gemm_plan_meets_the_contract(m, k, n):
    w, x, ref = _gemm_case(m, k, n)
    wt = affine_to_torch(w, "bf16")
    xt = act_to_torch(x, "bf16")
    cands = tuning.gemm_plan_candidates(m, k, n, 64)
    assert tuning.gemm_plan(m, k, n, 64, torch.bfloat16) in cands
    worst = 0.0
    for plan in cands:
        print(f"[gemm {m}x{k}x{n}] plan {plan}", flush=True)
        tuning.install_gemm_plan(m, k, n, 64, torch.bfloat16, plan)
        y = mt.affine_matmul(xt, *wt)
        torch.cuda.synchronize()
        worst = max(worst, _check(str(plan), torch_to_act(y, "bf16"), ref))
    print(f"[gemm {m}x{k}x{n}] {len(cands)} plans, worst tolerance_error {worst:.2e}", flush=True)


def test_tuner_decides_persists_and_reloads(monkeypatch, tmp_path):
    monkeypatch.setenv("METILE_AMD_CACHE_DIR", str(tmp_path))
    monkeypatch.delenv("METILE_AMD_DISABLE_TUNING", raising=False)
    gate = O.make_affine_weight(8960, 1536, 4, 64, 1, 10)
    up = O.make_affine_weight(8960, 1536, 4, 64, 1, 12)
    x = O.make_activations(1, 1536, 1)
    ref = O.affine_swiglu(x, gate, up, 64, 4)
    gt, ut = affine_to_torch(gate, "bf16"), affine_to_torch(up, "bf16")
    packed = (mt.affine_repack(gt[0]), gt[1], gt[2], mt.affine_repack(ut[0]), ut[1], ut[2])
    xt = act_to_torch(x, "bf16")
    planner = tuning.qmv_plan(1, 1536, 8960, 64, 4, 2, torch.bfloat16)

    decision = tuning.ensure_qmv_plans(xt, packed, group_size=64, bits=4)
    entries = tuning.load_decisions()
    assert len(entries) == 1
    record = next(iter(entries.values()))
    print(f"[tuner swiglu M=1] planner {record['planner']} {record['planner_us']} us, "
          f"chosen {record['plan']} {record['chosen_us']} us, {record['copies']} weight copies",
          flush=True)
    assert record["planner"] == tuning.asdict(planner)
    assert 0 < record["chosen_us"] <= record["planner_us"]
    plan = decision[1]
    installed = tuning.qmv_plan(1, 1536, 8960, 64, 4, 2, torch.bfloat16)
    assert installed == (plan if plan is not None else planner)
    _check("tuned swiglu", torch_to_act(mt.mlx_affine_swiglu(xt, *gt, *ut), "bf16"), ref)
    (seen,) = mt.mlx_affine_swiglu_dispatches()
    assert (seen["rows"], seen["source"]) == (1, "measured")
    assert tuning.QmvPlan(seen["kernel"], seen["ksplit"], seen["strips"], seen["tiles"],
                          seen["order"]) == installed

    # a fresh process state: the decision comes back from the cache, no measuring
    tuning.clear_plans()
    monkeypatch.setenv("METILE_AMD_DISABLE_TUNING", "1")
    assert tuning.ensure_qmv_plans(xt, packed, group_size=64, bits=4) == decision
    assert tuning.qmv_plan(1, 1536, 8960, 64, 4, 2, torch.bfloat16) == installed
    assert [d["source"] for d in mt.mlx_affine_swiglu_dispatches()] == ["cached"]
    # decisions apply to both code layouts: MLX codes give the same bits as repacked ones
    assert _same(mt.affine_swiglu(xt, *gt, *ut), mt.affine_swiglu(xt, *packed))


def test_layout_decision_persists_and_reloads(monkeypatch, tmp_path):
    # the down projection at M=1: plans over both code layouts, the fastest pair kept
    monkeypatch.setenv("METILE_AMD_CACHE_DIR", str(tmp_path))
    monkeypatch.delenv("METILE_AMD_DISABLE_TUNING", raising=False)
    down = O.make_affine_weight(1536, 8960, 4, 64, 3, 14)
    h = O.make_activations(1, 8960, 3)
    res = O.make_activations(1, 1536, 3, tensor_id=3)
    ref = O.affine_qmv(h, *down, 64, 4, residual=res)
    mlx = affine_to_torch(down, "bf16")
    packed = (mt.affine_repack(mlx[0]), mlx[1], mlx[2])
    ht, rt = act_to_torch(h, "bf16"), act_to_torch(res, "bf16")
    layouts = {"repacked": packed, "mlx": mlx}
    layout = tuning.ensure_qmv_layout(ht, layouts, group_size=64, bits=4)
    assert layout in layouts
    (seen,) = mt.mlx_affine_residual_qmv_dispatches()
    assert (seen["rows"], seen["layout"], seen["source"]) == (1, layout, "measured")
    entries = tuning.load_decisions()
    assert len(entries) == 1
    record = next(iter(entries.values()))
    print(f"[tuner down M=1 layouts] planner {record['planner']} {record['planner_us']} us "
          f"(repacked), chosen {record['plan']} {record['chosen_us']} us over {record['layout']}",
          flush=True)
    assert record["op"] == "affine_qmv_layout" and record["layout"] == layout
    assert 0 < record["chosen_us"] <= record["planner_us"]
    installed = tuning.qmv_plan(1, 8960, 1536, 64, 4, 1, torch.bfloat16)
    a = mt.affine_qmv(ht, *layouts[layout], residual=rt)
    b = mt.affine_qmv(ht, *layouts["mlx" if layout == "repacked" else "repacked"], residual=rt)
    assert _same(a, b)
    _check("layout-tuned down", torch_to_act(a, "bf16"), ref)
    # a fresh process state: plan and layout come back from the cache, no measuring
    tuning.clear_plans()
    monkeypatch.setenv("METILE_AMD_DISABLE_TUNING", "1")
    assert tuning.ensure_qmv_layout(ht, layouts, group_size=64, bits=4) == layout
    assert tuning.qmv_plan(1, 8960, 1536, 64, 4, 1, torch.bfloat16) == installed


def test_tuned_executor_and_gemm(monkeypatch, tmp_path):
    monkeypatch.setenv("METILE_AMD_CACHE_DIR", str(tmp_path))
    monkeypatch.delenv("METILE_AMD_DISABLE_TUNING", raising=False)
    # an MLP executor at Qwen2.5-0.5B shape (hidden 896, intermediate 4864), 3 rows
    gate = O.make_affine_weight(4864, 896, 4, 64, 2, 10)
    up = O.make_affine_weight(4864, 896, 4, 64, 2, 12)
    down = O.make_affine_weight(896, 4864, 4, 64, 2, 14)
    x = O.make_activations(3, 896, 2)
    res = O.make_activations(3, 896, 2, tensor_id=3)
    ref, _ = O.affine_mlp(x, gate, up, down, 64, 4, residual=res)
    xt, rt = act_to_torch(x, "bf16"), act_to_torch(res, "bf16")
    ts = [affine_to_torch(w, "bf16") for w in (gate, up, down)]
    ex = mt.mlx_affine_mlp_executor(xt, *ts[0], *ts[1], *ts[2], rt)
    _check("tuned mlp", torch_to_act(ex(xt, rt), "bf16"), ref, min_exact=0.85)
    entries = tuning.load_decisions()
    assert {e["nproj"] for e in entries.values()} == {1, 2}  # both stages decided
    assert all(e["layout"] in ("mlx", "repacked") for e in entries.values())
    # a one-row call: its row bucket gets its own plans and layouts on first use
    ref1, _ = O.affine_mlp(x[:1], gate, up, down, 64, 4, residual=res[:1])
    _check("tuned mlp, one row", torch_to_act(ex(xt[:1], rt[:1]), "bf16"), ref1, min_exact=0.85)
    rows = {(e["rows"], e["nproj"]) for e in tuning.load_decisions().values()}
    assert {(1, 1), (1, 2), (4, 1), (4, 2)} <= rows
    # the executor's decisions, as the reference's dispatch introspection lists them
    for seen, nproj in ((mt.mlx_affine_swiglu_dispatches(), 2),
                        (mt.mlx_affine_residual_qmv_dispatches(), 1)):
        assert {d["rows"] for d in seen} == {1, 4}
        assert all(d["source"] == "measured" and d["layout"] in ("mlx", "repacked")
                   for d in seen if d["rows"] == 4)
        assert all(tuning.QmvPlan(d["kernel"], d["ksplit"], d["strips"], d["tiles"], d["order"])
                   == tuning.qmv_plan(d["rows"], d["input_features"], d["output_features"], 64,
                                      4, nproj, torch.bfloat16) for d in seen)
    # the prefill GEMM through the tuned reference entry
    w = affine_to_torch(O.make_affine_weight(1536, 1024, 4, 64, 9, 10), "bf16")
    aw = mt.AffineWeight.from_torch(*w)
    xp = act_to_torch(O.make_activations(200, 1024, 9), "bf16")
    y = mt.mlx_affine_matmul(xp, aw)
    assert mt.accuracy_compatible(y, mt.native_affine_matmul(xp, aw))
    gemm = [e for e in tuning.load_decisions().values()
            if e["op"] == "affine_matmul"]
    assert len(gemm) == 1
    (seen,) = mt.mlx_affine_matmul_dispatches()
    assert (seen["rows"], seen["input_features"], seen["output_features"], seen["source"]) == (
        256, 1024, 1536, "measured")
    assert tuning.GemmPlan(seen["kernel"], seen["tile_m"], seen["tile_n"], seen["ksplit"],
                           seen["order"]) == tuning.gemm_plan(
        200, 1024, 1536, 64, torch.bfloat16)
    print(f"[tuner gemm 200x1024x1536] planner {gemm[0]['planner']} {gemm[0]['planner_us']} us, "
          f"chosen {gemm[0]['plan']} {gemm[0]['chosen_us']} us", flush=True)
