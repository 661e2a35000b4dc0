"""The tuner's host side, no GPU: the decision log and keys, the screening order, the ABBA
head-to-head arithmetic and its tail-quantile ranking, the selection rule, and the plan table of
the C ABI (candidate lists, validation, installation, bucketing, workspace sizes), which is
host-only code.

The tuner fills the role of ``metile/runtime/cache.py:12-56`` and
``metile/tuning/tournament.py:21-94`` with its own design (an append-only, locked decision
log; shuffled screening; ABBA pairs); the selection rule is this build's (a margin over the
planner's plan, ties to the fewest workgroups)."""

from __future__ import annotations

import json
import multiprocessing
import os

import pytest
import torch

import metile_amd._lib as L
from metile_amd import build, tuning
from metile_amd.tuning import DensePlan, GemmPlan, QmvPlan


# ---- decision log --------------------------------------------------------------------------------


def test_cache_dir_precedence(monkeypatch, tmp_path):
    monkeypatch.setenv("METILE_AMD_CACHE_DIR", str(tmp_path / "a"))
    monkeypatch.setenv("XDG_CACHE_HOME", str(tmp_path / "x"))
    assert tuning.cache_dir() == tmp_path / "a"
    monkeypatch.delenv("METILE_AMD_CACHE_DIR")
    assert tuning.cache_dir() == tmp_path / "x" / "metile_amd"
    monkeypatch.delenv("XDG_CACHE_HOME")
    assert tuning.cache_dir().parts[-2:] == (".cache", "metile_amd")


def test_decision_key_is_readable_and_hashes_the_context():
    shape = {"rows": 1, "input_features": 1536}
    a = tuning.decision_key("affine_qmv", shape, ("lib", [1, 2]))
    assert a.startswith("affine_qmv:input_features=1536,rows=1#") and len(a.split("#")[1]) == 24
    assert a == tuning.decision_key("affine_qmv", dict(reversed(list(shape.items()))),
                                    ("lib", [1, 2]))
    assert a != tuning.decision_key("affine_qmv", shape, ("lib", [2, 1]))
    assert a != tuning.decision_key("affine_matmul", shape, ("lib", [1, 2]))


def test_log_appends_last_entry_wins_and_skips_torn_lines(tmp_path):
    path = tmp_path / "d" / "log.jsonl"
    assert tuning.load_decisions(path) == {}
    tuning.append_decision("k", {"plan": None}, path)
    tuning.append_decision("j", {"plan": {"tile": 64}}, path)
    tuning.append_decision("k", {"plan": {"tile": 128}}, path)
    with open(path, "a") as f:
        f.write('{"key": "torn", "entry"')  # a line cut short
    assert tuning.load_decisions(path) == {"k": {"plan": {"tile": 128}},
                                           "j": {"plan": {"tile": 64}}}
    assert len(path.read_text().splitlines()) == 4  # appended, never rewritten


def _append_many(args):
    path, who = args
    for i in range(50):
        tuning.append_decision(f"{who}-{i}", {"plan": None, "i": i}, path)


def test_concurrent_writers_keep_every_decision(tmp_path):
    path = tmp_path / "log.jsonl"
    with multiprocessing.get_context("spawn").Pool(4) as pool:
        pool.map(_append_many, [(path, w) for w in range(4)])
    got = tuning.load_decisions(path)
    assert len(got) == 200 and all(got[f"{w}-{i}"]["i"] == i for w in range(4) for i in range(50))


def test_decisions_round_trip_through_the_log(monkeypatch, tmp_path):
    monkeypatch.setenv("METILE_AMD_CACHE_DIR", str(tmp_path))
    plan = QmvPlan("staged", 3, 544, 1)
    tuning._write_decision("k1", plan, {"planner_us": 9.0})
    tuning._write_decision("k2", None, {"planner_us": 5.0})
    assert tuning._read_decision("k1", QmvPlan) == (True, plan)
    assert tuning._read_decision("k2", QmvPlan) == (True, None)
    assert tuning._read_decision("k3", QmvPlan) == (False, None)
    tuning.append_decision("k4", {"plan": {"tile": 64}})  # malformed: missing a field
    assert tuning._read_decision("k4", GemmPlan) == (False, None)
    assert {e.get("planner_us") for e in tuning.cached_decisions()} == {9.0, 5.0, None}
    monkeypatch.setenv("METILE_AMD_DISABLE_DISK_CACHE", "1")
    assert tuning._read_decision("k1", QmvPlan) == (False, None)
    tuning._write_decision("k5", plan, {})
    monkeypatch.delenv("METILE_AMD_DISABLE_DISK_CACHE")
    assert tuning._read_decision("k5", QmvPlan) == (False, None)


def test_row_bucket_and_dispatch_rows():
    assert [tuning.row_bucket(r) for r in (1, 2, 3, 5, 8, 9, 17, 32)] == [1, 2, 4, 8, 8, 16, 32,
                                                                         32]
    assert tuning.dispatch_rows(1, 64) == [1]
    assert tuning.dispatch_rows(32, 64) == [32]
    assert tuning.dispatch_rows(64, 64) == [32]
    assert tuning.dispatch_rows(70, 64) == [32, 6]
    assert tuning.dispatch_rows(20, 32) == [16, 4]
    assert tuning.dispatch_rows(48, 32) == [16]


# ---- timing and ranking --------------------------------------------------------------------------


def test_tail_quantile_interpolates_order_statistics():
    assert tuning.tail_quantile([4.0, 1.0, 3.0, 2.0, 5.0]) == 4.0
    assert tuning.tail_quantile([1.0, 2.0], 0.75) == pytest.approx(1.75)
    assert tuning.tail_quantile([7.0]) == 7.0
    with pytest.raises(ValueError):
        tuning.tail_quantile([])


def test_tail_quantile_rejects_a_bimodal_kernel_the_median_would_pick():
    """The case that motivates ranking on a tail (metile/tuning/tournament.py:21-42): a kernel
    quick when conditions line up (1643 us) but slower most of the time (2874 us) against a
    steady baseline (2047-2073 us). Its median beats the baseline; its upper quantile does
    not, and the baseline is kept."""
    bimodal = [1643.0, 1650.0, 1700.0, 1800.0, 2874.0, 2874.0, 2900.0]
    steady = [2047.0, 2052.0, 2060.0, 2066.0, 2073.0, 2050.0, 2061.0]
    med = {"base": sorted(steady)[3], "x": sorted(bimodal)[3]}
    assert tuning.choose(med, "base", lambda k: 0) == "x"  # what a median ranking would do
    tail = {"base": tuning.tail_quantile(steady), "x": tuning.tail_quantile(bimodal)}
    assert tuning.choose(tail, "base", lambda k: 0) == "base"


def test_screen_shuffles_each_round_and_times_everyone():
    order = []
    cands = [(k, k) for k in "abcdef"]
    samples = tuning.screen(cands, 6, lambda r: order.append(r) or float(len(order)))
    rounds = [order[i:i + 6] for i in range(0, 36, 6)]
    assert all(sorted(r) == list("abcdef") for r in rounds)
    assert len({tuple(r) for r in rounds}) > 1  # not one fixed order
    assert {k: len(v) for k, v in samples.items()} == dict.fromkeys("abcdef", 6)
    again = []
    tuning.screen(cands, 6, lambda r: again.append(r) or 0.0)
    assert again == order  # seeded: reproducible


def test_head_to_head_runs_abba_and_cancels_linear_drift():
    calls = []
    times = {"base": 10.0, "x": 8.0, "y": 12.0}

    def measure(r):
        calls.append(r)
        return times[r] * (1.0 + 0.01 * len(calls))  # a clock that drifts linearly

    got = tuning.head_to_head([("base", "base"), ("x", "x"), ("y", "y")], "base", 3, measure)
    assert calls[:4] == ["base", "x", "x", "base"]
    assert len(calls) == 2 * 3 * 4
    # ABBA: the drift of each block cancels in (c0 + c1) / (b0 + b1)
    ref = got["base"]
    assert got["x"] / ref == pytest.approx(0.8, rel=1e-12)
    assert got["y"] / ref == pytest.approx(1.2, rel=1e-12)


def test_choose_needs_the_margin_and_breaks_ties_by_cost():
    cost = {"base": 0, "a": 10, "b": 5, "c": 1}.__getitem__
    assert tuning.choose({"base": 100.0, "a": 99.0}, "base", cost) == "base"  # 1% < margin
    assert tuning.choose({"base": 100.0, "a": 95.0}, "base", cost) == "a"
    # a and b within the tie tolerance (1.5%): fewer workgroups wins; c is not tied
    assert tuning.choose({"base": 100.0, "a": 90.0, "b": 91.2, "c": 93.0}, "base", cost) == "b"
    assert tuning.choose({"base": 100.0, "a": 90.0, "b": 92.0}, "base", cost) == "a"
    # equal cost within the tolerance: the first by text, whichever measured faster
    same = {"base": 0, "p2": 3, "p1": 3}.__getitem__
    assert tuning.choose({"base": 100.0, "p1": 90.5, "p2": 90.0}, "base", same) == "p1"
    assert tuning.choose({"base": 100.0, "p1": 90.0, "p2": 90.5}, "base", same) == "p1"


# ---- the plan table of the C ABI (host-only) -----------------------------------------------------

SHAPES = [  # (rows, K, N, group, bits, nproj)
    (1, 1536, 8960, 64, 4, 2), (1, 8960, 1536, 64, 4, 1), (16, 1536, 8960, 64, 4, 2),
    (32, 1536, 8960, 64, 4, 1), (1, 5120, 17408, 64, 8, 1), (3, 1024, 1536, 32, 8, 2),
    (8, 896, 4864, 64, 4, 2), (4, 4864, 896, 64, 4, 1),
]


@pytest.fixture
def clean_plans():
    tuning.clear_plans()
    yield
    tuning.clear_plans()


@pytest.mark.parametrize("shape", SHAPES)
def test_candidates_are_valid_and_include_the_planner(shape, clean_plans):
    rows, k, n, g, bits, nproj = shape
    cands = tuning.qmv_plan_candidates(rows, k, n, g, bits, nproj)
    assert cands and len(set(cands)) == len(cands)
    import torch

    for dtype in (torch.bfloat16, torch.float16):
        planner = tuning.qmv_plan(rows, k, n, g, bits, nproj, dtype)
        if tuning.row_bucket(rows) == rows:
            assert planner in cands
    gemv = [c for c in cands if c.kernel == "gemv"]
    # GEMV plans exist for up to 4 rows: 2, 4 and 8 columns per group, and for each number of
    # passes over K's 16-byte chunks the fewest waves (of 64 lanes) that make it; with more
    # than one pass, at most 8 of projections x columns x rows (registers)
    bucket = tuning.row_bucket(rows)
    chunks = k * bits // 128

    def groups(w):  # column groups per workgroup
        if chunks <= 64:  # whole groups in every wave
            return w * (64 // chunks if chunks % 16 == 0 else 1)
        return 64 * w // chunks if chunks <= 64 * w and chunks % 16 == 0 else 1

    if chunks <= 64:
        waves = set(range(1, 9))
    else:
        waves = {-(-chunks // (64 * p)) for p in range(1, 17)} & set(range(1, 9))
        waves |= {w for w in range(1, 9) if groups(w) >= 2 and 64 * w % chunks == 0}

    def fits(c, w):
        one_pass = chunks <= 64 * w
        if c == 8:  # eight columns: one projection of up to two rows, in one pass
            return one_pass and nproj == 1 and bucket <= 2
        return one_pass or nproj * c * min(bucket, 4) <= 8

    # ... each in both workgroup orders; a workgroup covers groups(w) groups of c columns
    assert sorted((c.strips, c.tiles, c.order) for c in gemv) == (
        sorted((n // (c * groups(w)), w, o) for c in (2, 4, 8) for w in waves for o in (0, 1)
               if fits(c, w) and n % (c * groups(w)) == 0)
        if bucket <= 4 else [])
    # column blocks: one or two workgroups per CU (256 CUs on the host, with no device), or
    # blocks of 16 or 32 columns, at most 64 wide in either code layout; 4, 6 or 8 waves; K unsplit
    # or in 4 equal splits; groups of 64 or more
    align = 16 // bits
    # the 4x4x4-MFMA GEMV: up to 4 rows of 4-bit codes, 1, 2 or 4 groups of 4 columns per
    # workgroup, every wave count that gives each wave one to four 512-wide K rounds whose loads
    # (4 + 3 nproj groups each) stay below 64
    rounds = -(-k // 512)
    assert sorted((c.strips, c.tiles) for c in cands if c.kernel == "gemv4") == (
        sorted((n // (4 * cg), w) for cg in (1, 2, 4) for w in range(1, 9)
               if w <= rounds and -(-rounds // w) <= 4
               and -(-rounds // w) * (4 + 3 * nproj * cg) < 64 and n % (4 * cg) == 0)
        if bucket <= 4 and bits == 4 else [])
    for c in cands:
        assert c.kernel in ("staged", "register", "gemv", "block", "gemv4")
        if c.kernel == "gemv4":
            assert c.ksplit == 1 and c.strips in (n // 4, n // 8, n // 16) and c.order == 0
        elif c.kernel == "register":
            assert g != 32 and c.strips == n // 32 and c.tiles == 1
        elif c.kernel == "gemv":
            assert c.ksplit == 1 and c.workgroups == c.strips
        elif c.kernel == "block":
            assert g >= 64 and rows <= 32 and c.order == 0
            assert c.ksplit in (1, 4) and c.tiles in (4, 6, 8)
            assert c.strips in (256, 512, n // 16, n // 32)
            assert max(-(-n // c.strips), -(-(n // align) // c.strips) * align) <= 64
        else:
            assert rows <= (16 if g == 32 else 32)
            assert n // 32 <= c.strips <= 2 * (n // 32) and c.strips % c.tiles == 0
        tuning.install_qmv_plan(rows, k, n, g, bits, nproj, torch.bfloat16, c)
        assert tuning.qmv_plan(rows, k, n, g, bits, nproj, torch.bfloat16) == c


def test_installed_plans_are_bucketed_per_dtype_and_size_the_workspace(clean_plans):
    import torch

    lib = L.lib()
    k, n = 8960, 1536
    planner = tuning.qmv_plan(5, k, n, 64, 4, 1, torch.bfloat16)
    before = lib.mt_affine_qmv_workspace_bytes(5, k, n, 64, 4, 1)
    wide = max(tuning.qmv_plan_candidates(5, k, n, 64, 4, 1), key=lambda p: p.ksplit)
    assert wide.ksplit > planner.ksplit
    tuning.install_qmv_plan(5, k, n, 64, 4, 1, torch.bfloat16, wide)
    # rows 5..8 share the bucket; 4 and 9 do not; the other dtype keeps the planner's plan
    for rows in (5, 6, 8):
        assert tuning.qmv_plan(rows, k, n, 64, 4, 1, torch.bfloat16) == wide
    assert tuning.qmv_plan(4, k, n, 64, 4, 1, torch.bfloat16) != wide
    assert tuning.qmv_plan(9, k, n, 64, 4, 1, torch.bfloat16) != wide
    assert tuning.qmv_plan(5, k, n, 64, 4, 1, torch.float16) == planner
    # the workspace query covers the installed plan (more K splits, more partial sums)
    after = lib.mt_affine_qmv_workspace_bytes(5, k, n, 64, 4, 1)
    assert after == 64 * 1024 + wide.ksplit * 5 * n * 4 > before
    # a call of 37 rows runs a 32-row and a 5-row dispatch: both are covered
    assert lib.mt_affine_qmv_workspace_bytes(37, k, n, 64, 4, 1) >= after
    tuning.install_qmv_plan(5, k, n, 64, 4, 1, torch.bfloat16, None)
    assert tuning.qmv_plan(5, k, n, 64, 4, 1, torch.bfloat16) == planner
    assert lib.mt_affine_qmv_workspace_bytes(5, k, n, 64, 4, 1) == before


@pytest.mark.parametrize("plan,message", [
    (QmvPlan("staged", 1, 279, 1), "strips must be in N/32..2N/32"),
    (QmvPlan("staged", 1, 561, 1), "strips must be in N/32..2N/32"),
    (QmvPlan("staged", 1, 281, 2), "multiple of tiles"),
    (QmvPlan("staged", 1, 280, 3), "tiles must be 1 or 2"),
    (QmvPlan("register", 1, 300, 1), "N/32 strips"),
    (QmvPlan("register", 1, 280, 2), "N/32 strips"),
    (QmvPlan("staged", 0, 280, 1), "ksplit must be in 1..K/64"),
    (QmvPlan("staged", 25, 280, 1), "ksplit must be in 1..K/64"),
    (QmvPlan("staged", 7, 280, 1), "equal-length splits"),  # 24 steps in 7 splits is 6 of 4
    (QmvPlan("gemv", 2, 2240, 4), "does not split K"),
    (QmvPlan("gemv", 1, 1120, 1), "does not hold this many columns"),  # 8 columns, 2 proj
    (QmvPlan("gemv", 1, 560, 1), "GEMV strips must be"),    # 16 columns per workgroup
    (QmvPlan("gemv", 1, 1120, 5), "GEMV strips must be"),   # 5 waves: 5 groups of 48 chunks
    (QmvPlan("gemv", 1, 2240, 0), "in 1..8"),
    (QmvPlan("gemv", 1, 2240, 9), "in 1..8"),
    (QmvPlan("gemv", 1, 2240, 1, 2), "order must be 0 or 1"),
    (QmvPlan("staged", 1, 280, 1, 1), "order is a GEMV plan field"),
])
def test_invalid_qmv_plans_are_rejected(plan, message, clean_plans):
    import torch

    with pytest.raises(ValueError, match=message):
        tuning.install_qmv_plan(1, 1536, 8960, 64, 4, 2, torch.bfloat16, plan)
    assert tuning.qmv_plan(1, 1536, 8960, 64, 4, 2, torch.bfloat16) != plan


def test_plan_rules_that_depend_on_rows_and_groups(clean_plans):
    import torch

    # the staged kernel takes at most 32 rows (16 with groups of 32), within its LDS; the
    # register kernel no groups of 32
    with pytest.raises(ValueError, match="rows of one dispatch, at most 16"):
        tuning.install_qmv_plan(17, 1024, 1536, 32, 4, 1, torch.bfloat16,
                                QmvPlan("staged", 1, 48, 1))
    with pytest.raises(ValueError, match="LDS does not hold"):
        tuning.install_qmv_plan(17, 1536, 8960, 64, 4, 1, torch.bfloat16,
                                QmvPlan("staged", 1, 280, 1))
    tuning.install_qmv_plan(17, 1536, 8960, 64, 4, 2, torch.bfloat16, QmvPlan("staged", 1, 280, 2))
    with pytest.raises(ValueError, match="groups of 64 or more"):
        tuning.install_qmv_plan(1, 1024, 1536, 32, 8, 1, torch.bfloat16,
                                QmvPlan("register", 1, 48, 1))
    # the GEMV kernel takes at most 4 rows; with two passes over K (280 chunks per column, 128
    # lanes) at most 8 of projections x columns x rows; in one pass (48 chunks) any
    with pytest.raises(ValueError, match="more rows than the GEMV kernel"):
        tuning.install_qmv_plan(5, 8960, 1536, 64, 4, 1, torch.bfloat16,
                                QmvPlan("gemv", 1, 384, 4))
    with pytest.raises(ValueError, match="in registers"):
        tuning.install_qmv_plan(4, 8960, 1536, 64, 4, 1, torch.bfloat16,
                                QmvPlan("gemv", 1, 384, 2))
    tuning.install_qmv_plan(4, 8960, 1536, 64, 4, 1, torch.bfloat16, QmvPlan("gemv", 1, 768, 2))
    tuning.install_qmv_plan(4, 1536, 8960, 64, 4, 2, torch.bfloat16, QmvPlan("gemv", 1, 2240, 1))
    tuning.install_qmv_plan(4, 8960, 1536, 32, 8, 1, torch.bfloat16, QmvPlan("gemv", 1, 768, 8))
    # one dispatch holds at most 32 rows (16 with groups of 32)
    with pytest.raises(ValueError, match="rows of one dispatch"):
        tuning.qmv_plan(33, 1536, 8960, 64, 4, 1, torch.bfloat16)
    with pytest.raises(ValueError, match="rows of one dispatch"):
        tuning.qmv_plan(17, 1024, 1536, 32, 8, 1, torch.bfloat16)
    # every split holds fewer than 64 groups: 140 steps need at least 3 splits
    with pytest.raises(ValueError, match="too many groups per split"):
        tuning.install_qmv_plan(1, 8960, 1536, 64, 4, 1, torch.bfloat16,
                                QmvPlan("register", 2, 48, 1))
    # where one strip's staging does not fit, the planner takes two-strip workgroups before
    # another K split (one projection at 32 rows: unsplit; the down projection: the fewest
    # splits whose staging two strips hold, 6 of 24 steps each)
    assert tuning.qmv_plan(32, 1536, 8960, 64, 4, 1, torch.bfloat16) == QmvPlan("staged", 1, 280, 2)
    assert tuning.qmv_plan(32, 8960, 1536, 64, 4, 1, torch.bfloat16) == QmvPlan("staged", 6, 48, 2)
    assert tuning.qmv_plan(16, 8960, 1536, 64, 4, 1, torch.bfloat16) == QmvPlan("staged", 5, 48, 1)


def test_gemm_plans(clean_plans):
    import torch

    lib = L.lib()
    m, k, n = 512, 8960, 1536
    planner = tuning.gemm_plan(m, k, n, 64, torch.bfloat16)
    # the planner takes the ring kernel at config 4: 128 x 96 tiles in four splits (36 steps)
    # for the down projection, 128 x 192 tiles unsplit for the up projection
    assert planner == GemmPlan("ring", 128, 96, 4)
    assert tuning.gemm_plan(512, 1536, 8960, 64, torch.bfloat16) == GemmPlan("ring", 128, 192, 1, 2)
    cands = tuning.gemm_plan_candidates(m, k, n, 64)
    assert planner in cands
    assert {(c.kernel, c.tile_m, c.tile_n) for c in cands} == {
        ("staged", 64, 64), ("staged", 128, 128), ("ring", 128, 64), ("ring", 128, 96),
        ("ring", 128, 128), ("ring", 128, 160), ("ring", 128, 192), ("ring", 128, 256)}
    # every ring plan in the three tile orders, the register-staged ones in grid order only
    ring = [c for c in cands if c.kernel == "ring"]
    assert {c.order for c in ring} == {0, 1, 2} and len(ring) % 3 == 0
    assert all(GemmPlan(c.kernel, c.tile_m, c.tile_n, c.ksplit, o) in cands
               for c in ring for o in (0, 1, 2))
    assert all(c.order == 0 for c in cands if c.kernel == "staged")
    # ring splits are whole three-step lengths: 140 steps split 4 ways run 36 + 36 + 36 + 32
    assert GemmPlan("ring", 128, 64, 4) in cands and GemmPlan("ring", 128, 64, 3) in cands
    assert all(c.ksplit <= 8 for c in cands if c.kernel == "ring")
    before = lib.mt_affine_gemm_workspace_bytes(m, k, n, 64, 4)
    pick = next(c for c in cands if c.ksplit == 8 and c.kernel == "staged" and c.tile_m == 64)
    tuning.install_gemm_plan(m, k, n, 64, torch.bfloat16, pick)
    assert tuning.gemm_plan(300, k, n, 64, torch.bfloat16) == pick  # same bucket (512)
    assert tuning.gemm_plan(m, k, n, 64, torch.float16) == planner
    # the workspace serves either dtype: bf16 takes 8 splits now, f16 the planner's 4
    assert lib.mt_affine_gemm_workspace_bytes(m, k, n, 64, 4) == 64 * 1024 + 8 * m * n * 4
    tuning.install_gemm_plan(m, k, n, 64, torch.bfloat16, GemmPlan("ring", 128, 96, 2))
    assert lib.mt_affine_gemm_workspace_bytes(m, k, n, 64, 4) == 64 * 1024 + 4 * m * n * 4
    tuning.install_gemm_plan(m, k, n, 64, torch.bfloat16, pick)
    for bad, why in ((GemmPlan("staged", 96, 96, 1), "kernel 0 takes square tiles"),
                     (GemmPlan("staged", 128, 64, 1), "kernel 0 takes square tiles"),
                     (GemmPlan("ring", 128, 224, 1), "kernel 1 takes tiles of 128 x"),
                     (GemmPlan("ring", 64, 64, 1), "kernel 1 takes tiles of 128 x"),
                     (GemmPlan("ring", 128, 64, 9), "at most 8 K splits"),
                     (GemmPlan("ring", 128, 96, 4, 3), "order must be 0, 1 or 2"),
                     (GemmPlan("staged", 128, 128, 1, 1), "kernel 0 takes order 0")):
        with pytest.raises(ValueError, match=why):
            tuning.install_gemm_plan(m, k, n, 64, torch.bfloat16, bad)
    # 24 steps in five splits: lengths of 6 (whole three-step iterations) give only four
    with pytest.raises(ValueError, match="whole three-step iterations"):
        tuning.install_gemm_plan(m, 1536, 8960, 64, torch.bfloat16, GemmPlan("ring", 128, 160, 5))
    tuning.clear_plans()
    assert tuning.gemm_plan(m, k, n, 64, torch.bfloat16) == planner
    assert lib.mt_affine_gemm_workspace_bytes(m, k, n, 64, 4) == before


def test_dispatches_report_every_resolved_shape(clean_plans):
    """The reference's ``*_dispatches()`` introspection (``mlx_quantized.py:1627,1835``,
    ``mlx_affine.py:409``): one record per resolved shape, its plan as the library runs it
    now (a decided plan, else the planner's), sorted by shape, cleared with the plans."""
    import metile_amd as mt

    bf = torch.bfloat16
    swiglu = ("qmv", 0, 1, 1536, 8960, 64, 4, 2, bf)
    down = ("qmv", 0, 16, 8960, 1536, 64, 4, 1, bf)
    down1 = ("qmv", 0, 1, 8960, 1536, 64, 4, 1, bf)
    gemm = ("gemm", 0, 512, 1536, 8960, 64, bf)
    with tuning._lock:
        tuning._resolved.update({swiglu: "measured", down: "planner", down1: "cached",
                                 gemm: "cached"})
        tuning._decided[swiglu] = QmvPlan("gemv", 1, 2240, 2, 1)
        tuning._decided[down1] = QmvPlan("gemv", 1, 768, 5, 1)
        tuning._decided_layouts[(*swiglu, ("repacked", "mlx"))] = (tuning._decided[swiglu],
                                                                   "mlx")
        tuning._decided[gemm] = GemmPlan("ring", 128, 160, 1)

    (sw,) = mt.mlx_affine_swiglu_dispatches()
    assert sw == {"rows": 1, "input_features": 1536, "output_features": 8960,
                  "dtype": "torch.bfloat16", "group_size": 64, "bits": 4, "device": 0,
                  "kernel": "gemv", "ksplit": 1, "strips": 2240, "tiles": 2, "order": 1,
                  "layout": "mlx", "source": "measured"}
    qmv = mt.mlx_affine_residual_qmv_dispatches()
    assert [(d["rows"], d["source"], d["layout"]) for d in qmv] == [(1, "cached", None),
                                                                   (16, "planner", None)]
    planner = tuning.qmv_plan(16, 8960, 1536, 64, 4, 1, bf)
    assert (qmv[1]["kernel"], qmv[1]["ksplit"], qmv[1]["strips"], qmv[1]["tiles"]) == (
        planner.kernel, planner.ksplit, planner.strips, planner.tiles)
    assert qmv[0]["kernel"] == "gemv" and qmv[0]["strips"] == 768
    (mm,) = mt.mlx_affine_matmul_dispatches()
    assert (mm["rows"], mm["kernel"], mm["tile_m"], mm["tile_n"], mm["ksplit"], mm["source"]) == (
        512, "ring", 128, 160, 1, "cached")
    with pytest.raises(ValueError, match="op must be"):
        tuning.dispatches("dense")
    tuning.clear_plans()
    assert tuning.dispatches("swiglu") == tuning.dispatches("qmv") == () == \
        tuning.dispatches("matmul")


def test_candidate_buffer_contract():
    lib = L.lib()
    count = lib.mt_affine_qmv_plan_candidates(1, 1536, 8960, 64, 4, 2, None, 0)
    assert count > 0
    buf = (L.QmvPlan * 2)()
    assert lib.mt_affine_qmv_plan_candidates(1, 1536, 8960, 64, 4, 2, buf, 2) == count
    assert lib.mt_affine_qmv_plan_candidates(1, 1536, 8960, 64, 4, 2, None, 5) == \
        L.MT_ERR_INVALID_ARGUMENT
    assert lib.mt_affine_qmv_plan(1, 1536, 8960, 64, 4, 2, 0, None) == L.MT_ERR_INVALID_ARGUMENT
    assert lib.mt_affine_qmv_plan_candidates(1, 1500, 8960, 64, 4, 2, None, 0) == \
        L.MT_ERR_INVALID_ARGUMENT  # K not a multiple of 64
    assert lib.mt_plans_clear() == L.MT_OK


def test_library_reports_the_digest_of_its_sources():
    digest = L.lib().mt_source_digest().decode()
    assert len(digest) == 64 and int(digest, 16) >= 0
    sources = [*build.sources(), *build.CSRC.glob("*.h"), *build.INCLUDE.glob("*.h")]
    if max(p.stat().st_mtime for p in sources) > build.LIB.stat().st_mtime:
        pytest.skip("a source changed after the library was built: rebuild to compare digests")
    assert digest == build.source_digest()


def test_layout_choice_argument_checks():
    # the layout map is validated before anything is measured (no GPU needed)
    import torch

    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    mlx = (torch.zeros(64, 16, dtype=torch.int32), torch.zeros(64, 2, dtype=torch.bfloat16),
           torch.zeros(64, 2, dtype=torch.bfloat16))
    packed = (torch.zeros(2, 64, 8, dtype=torch.int32), mlx[1], mlx[2])
    with pytest.raises(ValueError, match="layouts must map"):
        tuning.ensure_qmv_layout(x, {}, group_size=64, bits=4)
    with pytest.raises(ValueError, match="layouts must map"):
        tuning.ensure_qmv_layout(x, {"packed": packed, "mlx": mlx}, group_size=64, bits=4)
    with pytest.raises(ValueError, match="not in that layout"):
        tuning.ensure_qmv_layout(x, {"repacked": mlx, "mlx": packed}, group_size=64, bits=4)


# ---- dense plans (host-only) ---------------------------------------------------------------------


def test_dense_plans_are_keyed_by_shape_only_and_size_the_workspace(clean_plans):
    import torch

    lib = L.lib()
    k, n = 8192, 2048
    planner = tuning.dense_plan(k, n, 1, torch.bfloat16)
    cands = tuning.dense_plan_candidates(k, n, 1)
    # every split of 128 steps into equal runs of at least 4 steps, at most 16 candidates
    splits = sorted({-(-128 // -(-128 // ks)) for ks in range(1, 17)})
    assert [c.ksplit for c in cands] == splits
    assert planner in cands
    other = max(cands, key=lambda c: c.ksplit)
    before = lib.mt_dense_workspace_bytes(128, k, n, 1)
    tuning.install_dense_plan(k, n, 1, torch.bfloat16, other)
    assert tuning.dense_plan(k, n, 1, torch.bfloat16) == other
    assert tuning.dense_plan(k, n, 1, torch.float16) == planner     # per dtype
    assert tuning.dense_plan(k, n, 2, torch.bfloat16) != other or other == planner  # per nproj
    # the workspace covers the installed plan at any row count (two 64-row chunks above 64)
    assert lib.mt_dense_workspace_bytes(128, k, n, 1) == 64 * 1024 + other.ksplit * 128 * n * 4
    assert lib.mt_dense_workspace_bytes(1, k, n, 1) == 64 * 1024 + other.ksplit * 1 * n * 4
    tuning.install_dense_plan(k, n, 1, torch.bfloat16, None)
    assert tuning.dense_plan(k, n, 1, torch.bfloat16) == planner
    assert lib.mt_dense_workspace_bytes(128, k, n, 1) == before


@pytest.mark.parametrize("plan,message", [
    (DensePlan(0), "ksplit must be in"),
    (DensePlan(33), "ksplit must be in"),
    (DensePlan(9), "equal-length splits"),    # 32 steps in runs of 4 make 8 splits, not 9
    (DensePlan(16), "at least 4 K steps"),    # 32 steps in 16 splits of 2
])
def test_invalid_dense_plans_are_rejected(plan, message, clean_plans):
    import torch

    with pytest.raises(ValueError, match=message):
        tuning.install_dense_plan(2048, 8192, 2, torch.bfloat16, plan)


def test_dispatches_report_the_plan_of_the_dispatch_rows_not_the_bucket(clean_plans, monkeypatch,
                                                                       tmp_path):
    """A shape resolved with nothing decided reports the plan the library runs at the
    dispatch's own row count: the planner plans from the rows (two-strip workgroups from four
    rows), which can differ within one row bucket (3 and 4 rows share bucket 4)."""
    monkeypatch.setenv("METILE_AMD_CACHE_DIR", str(tmp_path))
    monkeypatch.setattr(tuning, "_device_identity", lambda device: {"architecture": "cpu-test"})
    bf = torch.bfloat16
    k, n = 1536, 8960
    assert tuning.qmv_plan(3, k, n, 64, 4, 2, bf) != tuning.qmv_plan(4, k, n, 64, 4, 2, bf)
    x = torch.zeros(3, k, dtype=bf)
    w = torch.zeros(n, k // 8, dtype=torch.int32)
    s = torch.zeros(n, k // 64, dtype=bf)
    assert tuning.ensure_qmv_plans(x, (w, s, s, w, s, s), group_size=64, bits=4,
                                   autotune=False) == {3: None}
    (d,) = tuning.dispatches("swiglu")
    got = QmvPlan(d["kernel"], d["ksplit"], d["strips"], d["tiles"], d["order"])
    assert (d["rows"], d["source"]) == (4, "planner")
    assert got == tuning.qmv_plan(3, k, n, 64, 4, 2, bf)


def test_gemv4_plans_are_checked(clean_plans):
    import torch

    for rows, k, n, bits, plan, why in (
            (5, 1536, 256, 4, QmvPlan("gemv4", 1, 64, 1), "more rows"),
            (1, 1536, 256, 8, QmvPlan("gemv4", 1, 64, 1), "4-bit codes"),
            (1, 1536, 256, 4, QmvPlan("gemv4", 2, 64, 1), "does not split K"),
            (1, 1536, 256, 4, QmvPlan("gemv4", 1, 8, 1), "N/4, N/8 or N/16 workgroups"),
            (1, 1536, 256, 4, QmvPlan("gemv4", 1, 64, 4), "rounds"),  # 3 rounds, 4 waves
            (1, 8960, 256, 4, QmvPlan("gemv4", 1, 64, 4), "rounds")):  # 18 rounds: 5 per wave
        with pytest.raises(ValueError, match=why):
            tuning.install_qmv_plan(rows, k, n, 64, bits, 1, torch.bfloat16, plan)
    ok = QmvPlan("gemv4", 1, 64, 3)
    tuning.install_qmv_plan(4, 1536, 256, 32, 4, 2, torch.bfloat16, ok)
    assert tuning.qmv_plan(3, 1536, 256, 32, 4, 2, torch.bfloat16) == ok
