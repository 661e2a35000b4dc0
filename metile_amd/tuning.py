"""Plan tuning with a persistent decision cache.

Every C-ABI call plans itself from its shape (split-K, column strips, kernel). The planner's rules
were measured at the BASELINE shapes; for any other shape this module measures the plans the
library lists for it (``mt_affine_qmv_plan_candidates``, ``mt_affine_gemm_plan_candidates``) and
installs the fastest (``mt_affine_*_plan_set``), so that later calls of that shape take it. The
decision is appended to a persistent log keyed by everything that can change it, the role the
reference's tuner and cache play (``metile/runtime/cache.py:12-56``; keys
``mlx_quantized.py:1393-1449``; tournament ``metile/tuning/tournament.py:21-94``; selection
``mlx_quantized.py:1225-1253,1275-1336``).

What differs from the reference, by design:

* The baseline every candidate must beat is the planner's own plan (the reference's is MLX's
  native kernel). A candidate replaces it only when it is faster by ``SWITCH_MARGIN``; within
  ``TIE_TOLERANCE`` of the fastest the plan with the fewest workgroups wins (fewer partial sums),
  the analogue of the reference's shortest-description tie break, and among those the first in
  a fixed order of the plans (their text), never the noisier time. The tolerance (1.5%) is wider
  than the run-to-run spread of one plan's time across boxes, so that near-equal plans resolve
  the same way from run to run, and profiles taken in another process time the same plan.
* Candidates are timed as the hot path runs: each plan's dispatches are captured once in a HIP
  graph over enough copies of the weights (``COLD_BYTES``, more than twice the 256 MB Infinity
  Cache) that every dispatch streams its weights from HBM, and the graphs are replayed in a
  shuffled order (``screen``), then the finalists head to head against the baseline in ABBA
  blocks (``head_to_head``); both rank on an upper quantile of the samples (``tail_quantile``).
* Every candidate's result must pass the reference tuner's fidelity gate
  (``affine_swiglu_compatible``) against the planner plan's result before it is timed.
* A weight can be held in either code layout (MLX rows, or ``affine_repack``'s step-major
  repack), and the fastest plan depends on it: ``ensure_qmv_layout`` measures every plan over
  every layout the caller holds and keeps the fastest pair (the plan is installed, the layout
  returned for the caller to keep), as the reference's executors choose between their repacked
  and plain schedules.

Environment: ``METILE_AMD_CACHE_DIR`` (cache directory), ``METILE_AMD_DISABLE_DISK_CACHE=1``
(neither read nor write decisions), ``METILE_AMD_DISABLE_TUNING=1`` (never measure; cached
decisions still apply).
"""

from __future__ import annotations

import ctypes
import fcntl
import hashlib
import json
import math
import os
import random
import statistics
import threading
from dataclasses import asdict, astuple, dataclass
from pathlib import Path

import torch

from . import _lib

TUNER_VERSION = 3
SWITCH_MARGIN = 0.02
TIE_TOLERANCE = 0.015
FINALIST_SLACK = 1.10
TAIL_QUANTILE = 0.75
SCREEN_ROUNDS = 7
ABBA_BLOCKS = 8
COLD_BYTES = 600 << 20
MAX_COPIES = 256
CACHE_FILE = "affine-plans-v2.jsonl"

_LAYOUT_MLX, _LAYOUT_REPACKED = 0, 1
_LAYOUT_NAMES = {_LAYOUT_MLX: "mlx", _LAYOUT_REPACKED: "repacked"}
_KERNELS = {_lib.MT_QMV_STAGED: "staged", _lib.MT_QMV_REGISTER: "register",
            _lib.MT_QMV_GEMV: "gemv", _lib.MT_QMV_BLOCK: "block", _lib.MT_QMV_GEMV4: "gemv4"}
_KERNEL_CODES = {v: k for k, v in _KERNELS.items()}


# ---- decision log ------------------------------------------------------------------------------
# Decisions are appended, one JSON object per line, to a log that is never rewritten: the last
# line of a key wins. An append holds an exclusive lock on the file and a read a shared one
# (fcntl.flock), so tuning processes that share the cache keep each other's decisions, and a
# reader never sees half a line. Keys are readable (the op and the shape) with a short hash of
# everything else that can change the decision (the device, the library and tuner sources, the
# candidate list and the tuner's policy).


def cache_dir() -> Path:
    """``METILE_AMD_CACHE_DIR``, else ``$XDG_CACHE_HOME/metile_amd``, else
    ``~/.cache/metile_amd`` (not created here)."""
    explicit = os.environ.get("METILE_AMD_CACHE_DIR")
    if explicit:
        return Path(explicit).expanduser()
    base = os.environ.get("XDG_CACHE_HOME") or os.path.join(os.path.expanduser("~"), ".cache")
    return Path(base).expanduser() / "metile_amd"


def cache_path() -> Path:
    return cache_dir() / CACHE_FILE


def load_decisions(path: Path | None = None) -> dict:
    """``{key: entry}`` of the log at ``path`` (default ``cache_path()``), the last line of each
    key winning; lines that do not parse are skipped, a missing file reads as empty."""
    path = path or cache_path()
    try:
        f = open(path, "rb")
    except OSError:
        return {}
    out = {}
    with f:
        fcntl.flock(f.fileno(), fcntl.LOCK_SH)
        try:
            data = f.read()
        finally:
            fcntl.flock(f.fileno(), fcntl.LOCK_UN)
    for line in data.splitlines():
        try:
            rec = json.loads(line)
        except ValueError:
            continue
        if isinstance(rec, dict) and isinstance(rec.get("key"), str):
            out[rec["key"]] = rec.get("entry")
    return out


def append_decision(key: str, entry: dict, path: Path | None = None) -> None:
    """Append ``{key, entry}`` as one line under an exclusive lock."""
    path = path or cache_path()
    path.parent.mkdir(parents=True, exist_ok=True)
    line = json.dumps({"key": key, "entry": entry}, separators=(",", ":"), default=str) + "\n"
    fd = os.open(path, os.O_WRONLY | os.O_APPEND | os.O_CREAT, 0o644)
    try:
        fcntl.flock(fd, fcntl.LOCK_EX)
        try:
            os.write(fd, line.encode())
            os.fsync(fd)
        finally:
            fcntl.flock(fd, fcntl.LOCK_UN)
    finally:
        os.close(fd)


def decision_key(op: str, shape: dict, context) -> str:
    """``op:field=value,...#hash``: the shape in clear, ``context`` (anything else the decision
    depends on; its ``repr`` must be deterministic) as a 96-bit BLAKE2b hash."""
    h = hashlib.blake2b(digest_size=12)
    h.update(repr(context).encode())
    return op + ":" + ",".join(f"{k}={shape[k]}" for k in sorted(shape)) + "#" + h.hexdigest()


def disk_cache_enabled() -> bool:
    return os.environ.get("METILE_AMD_DISABLE_DISK_CACHE") != "1"


def tuning_enabled() -> bool:
    return os.environ.get("METILE_AMD_DISABLE_TUNING") != "1"


def row_bucket(rows: int) -> int:
    """The smallest power of two at or above ``rows`` (the library keys installed plans by it)."""
    bucket = 1
    while bucket < rows:
        bucket *= 2
    return bucket


# ---- plans ---------------------------------------------------------------------------------------


@dataclass(frozen=True)
class QmvPlan:
    """One small-row dispatch plan (``mt_qmv_plan``)."""

    kernel: str  # "staged", "register", "gemv", "block" or "gemv4" (4x4x4-MFMA GEMV)
    ksplit: int
    strips: int
    tiles: int = 1  # staged: strips per workgroup; gemv, block and gemv4: waves per workgroup
    order: int = 0  # gemv: 0 index order, 1 column groups dealt out XCD by XCD

    def to_c(self) -> _lib.QmvPlan:
        return _lib.QmvPlan(_KERNEL_CODES[self.kernel], self.ksplit, self.strips, self.tiles,
                            self.order)

    @classmethod
    def from_c(cls, p) -> "QmvPlan":
        return cls(_KERNELS[p.kernel], p.ksplit, p.strips, p.tiles, p.order)

    @property
    def workgroups(self) -> int:
        if self.kernel in ("gemv", "gemv4"):
            return self.strips
        if self.kernel == "block":
            return self.strips * self.ksplit
        return self.strips // self.tiles * self.ksplit


_GEMM_KERNELS = {_lib.MT_GEMM_STAGED: "staged", _lib.MT_GEMM_RING: "ring"}
_GEMM_KERNEL_CODES = {v: k for k, v in _GEMM_KERNELS.items()}


@dataclass(frozen=True)
class GemmPlan:
    """One prefill GEMM plan (``mt_gemm_plan``): the kernel ("staged": square tiles of 64 or
    128; "ring": tiles of 128 x 64 .. 256), its tile, the K splits and the tile order (ring:
    0 as launched, 1 / 2 each XCD a contiguous run of tiles, column tiles / row blocks fastest)."""

    kernel: str
    tile_m: int
    tile_n: int
    ksplit: int
    order: int = 0

    def to_c(self) -> _lib.GemmPlan:
        return _lib.GemmPlan(_GEMM_KERNEL_CODES[self.kernel], self.tile_m, self.tile_n,
                             self.ksplit, self.order)

    @classmethod
    def from_c(cls, p) -> "GemmPlan":
        return cls(_GEMM_KERNELS[p.kernel], p.tile_m, p.tile_n, p.ksplit, p.order)

    def workgroups(self, rows: int, n: int) -> int:
        return -(-rows // self.tile_m) * -(-n // self.tile_n) * self.ksplit


@dataclass(frozen=True)
class DensePlan:
    """One dense projection plan (``mt_dense_plan``): the K splits of every row count."""

    ksplit: int

    def to_c(self) -> _lib.DensePlan:
        return _lib.DensePlan(self.ksplit)

    @classmethod
    def from_c(cls, p) -> "DensePlan":
        return cls(p.ksplit)

    def workgroups(self, n: int) -> int:
        return n // 32 * self.ksplit


def _dtype_code(dtype) -> int:
    return {torch.bfloat16: _lib.MT_BF16, torch.float16: _lib.MT_F16}[dtype]


def qmv_plan(rows, k, n, group_size, bits, nproj, dtype) -> QmvPlan:
    """The plan a dispatch of ``rows`` rows takes now (installed, else the planner's)."""
    out = _lib.QmvPlan()
    _lib.check(_lib.lib().mt_affine_qmv_plan(rows, k, n, group_size, bits, nproj,
                                             _dtype_code(dtype), ctypes.byref(out)))
    return QmvPlan.from_c(out)


def qmv_plan_candidates(rows, k, n, group_size, bits, nproj) -> list[QmvPlan]:
    L = _lib.lib()
    count = L.mt_affine_qmv_plan_candidates(rows, k, n, group_size, bits, nproj, None, 0)
    if count < 0:
        _lib.check(count)
    buf = (_lib.QmvPlan * max(count, 1))()
    count = L.mt_affine_qmv_plan_candidates(rows, k, n, group_size, bits, nproj, buf, count)
    return [QmvPlan.from_c(buf[i]) for i in range(count)]


def install_qmv_plan(rows, k, n, group_size, bits, nproj, dtype, plan) -> None:
    """Install ``plan`` for the shape, both code layouts (``None`` restores the planner's)."""
    c = None if plan is None else ctypes.byref(plan.to_c())
    _lib.check(_lib.lib().mt_affine_qmv_plan_set(rows, k, n, group_size, bits, nproj,
                                                 _dtype_code(dtype), c))


def gemm_plan(rows, k, n, group_size, dtype) -> GemmPlan:
    out = _lib.GemmPlan()
    _lib.check(_lib.lib().mt_affine_gemm_plan(rows, k, n, group_size, _dtype_code(dtype),
                                              ctypes.byref(out)))
    return GemmPlan.from_c(out)


def gemm_plan_candidates(rows, k, n, group_size) -> list[GemmPlan]:
    L = _lib.lib()
    count = L.mt_affine_gemm_plan_candidates(rows, k, n, group_size, None, 0)
    if count < 0:
        _lib.check(count)
    buf = (_lib.GemmPlan * max(count, 1))()
    count = L.mt_affine_gemm_plan_candidates(rows, k, n, group_size, buf, count)
    return [GemmPlan.from_c(buf[i]) for i in range(count)]


def install_gemm_plan(rows, k, n, group_size, dtype, plan) -> None:
    c = None if plan is None else ctypes.byref(plan.to_c())
    _lib.check(_lib.lib().mt_affine_gemm_plan_set(rows, k, n, group_size, _dtype_code(dtype), c))


def dense_plan(k, n, nproj, dtype) -> DensePlan:
    """The plan every dense dispatch of this shape takes now (installed, else the planner's)."""
    out = _lib.DensePlan()
    _lib.check(_lib.lib().mt_dense_qmv_plan(k, n, nproj, _dtype_code(dtype), ctypes.byref(out)))
    return DensePlan.from_c(out)


def dense_plan_candidates(k, n, nproj) -> list[DensePlan]:
    L = _lib.lib()
    count = L.mt_dense_qmv_plan_candidates(k, n, nproj, None, 0)
    if count < 0:
        _lib.check(count)
    buf = (_lib.DensePlan * max(count, 1))()
    count = L.mt_dense_qmv_plan_candidates(k, n, nproj, buf, count)
    return [DensePlan.from_c(buf[i]) for i in range(count)]


def install_dense_plan(k, n, nproj, dtype, plan) -> None:
    c = None if plan is None else ctypes.byref(plan.to_c())
    _lib.check(_lib.lib().mt_dense_qmv_plan_set(k, n, nproj, _dtype_code(dtype), c))


def clear_plans() -> None:
    """Remove every installed plan and forget this process's decisions (the disk cache stays)."""
    with _lock:
        _lib.check(_lib.lib().mt_plans_clear())
        _decided.clear()
        _decided_layouts.clear()
        _resolved.clear()
        _planner_seen.clear()


# ---- timing and ranking -------------------------------------------------------------------------
# Screening replays every candidate once per round in a fresh random order (a fixed seed per
# round), so that no candidate keeps a place or a neighbour. The decision then times each
# finalist against the baseline alone, in ABBA order (baseline, candidate, candidate, baseline:
# a drift that is linear over the four cancels), and takes the candidate's time relative to
# the baseline in each block. Both stages rank on an upper quantile (TAIL_QUANTILE) of the
# samples rather than their median: a kernel that is fast when conditions line up but slow
# most of the time must not win on its good samples.


def tail_quantile(samples, q=None) -> float:
    """The ``q`` quantile (default ``TAIL_QUANTILE``) of ``samples``, interpolating linearly
    between order statistics."""
    q = TAIL_QUANTILE if q is None else q
    values = sorted(samples)
    if not values:
        raise ValueError("tail_quantile of no samples")
    pos = q * (len(values) - 1)
    i = math.floor(pos)
    j = min(i + 1, len(values) - 1)
    return values[i] + (values[j] - values[i]) * (pos - i)


def screen(candidates, rounds, measure, seed=0):
    """``{key: [seconds, ...]}``: each ``(key, runner)`` timed once per round, in an order
    shuffled anew every round."""
    items = list(candidates)
    samples = {key: [] for key, _ in items}
    rng = random.Random(seed)
    for _ in range(rounds):
        order = items[:]
        rng.shuffle(order)
        for key, runner in order:
            samples[key].append(measure(runner))
    return samples


def head_to_head(candidates, baseline, blocks, measure):
    """``{key: seconds}`` for the finalists ``candidates`` (which include ``baseline``): each
    other candidate is timed against the baseline alone in ``blocks`` ABBA blocks; its score is
    the tail quantile of its per-block time ratios to the baseline, given back in seconds as
    that ratio times the median of all the baseline's samples."""
    items = dict(candidates)
    base_runner = items[baseline]
    base_samples, ratios = [], {}
    for key, runner in items.items():
        if key == baseline:
            continue
        per_block = []
        for _ in range(blocks):
            b0 = measure(base_runner)
            c0 = measure(runner)
            c1 = measure(runner)
            b1 = measure(base_runner)
            base_samples += [b0, b1]
            per_block.append((c0 + c1) / (b0 + b1))
        ratios[key] = tail_quantile(per_block)
    if not base_samples:
        base_samples = [measure(base_runner) for _ in range(2 * blocks)]
    reference = statistics.median(base_samples)
    out = {baseline: reference}
    out.update({key: ratio * reference for key, ratio in ratios.items()})
    return out


def choose(timings, baseline, cost, *, margin=SWITCH_MARGIN, tie=TIE_TOLERANCE):
    """The key to install: the fastest of the candidates that beat ``baseline`` by ``margin``
    (within ``tie`` of the fastest, the lowest ``cost(key)``, then the first by ``repr``), else
    ``baseline``."""
    limit = timings[baseline] * (1.0 - margin)
    eligible = {k: t for k, t in timings.items() if k != baseline and t < limit}
    if not eligible:
        return baseline
    fastest = min(eligible.values())
    tied = [k for k, t in eligible.items() if t <= fastest * (1.0 + tie)]
    return min(tied, key=lambda k: (cost(k), repr(k)))


# ---- measuring plans on the GPU -----------------------------------------------------------------

_lock = threading.RLock()
_decided: dict[tuple, object] = {}
_decided_layouts: dict[tuple, tuple] = {}
# Every dispatch shape this process has resolved through ensure_qmv_plans, ensure_qmv_layout or
# ensure_gemm_plan, with how: "measured" (tuned now), "cached" (a disk decision) or "planner"
# (nothing decided: the library's own plan). Read by dispatches().
_resolved: dict[tuple, str] = {}
# The plan the library ran for a dispatch shape resolved with nothing decided, taken at that
# dispatch's own row count (the planner plans from the rows, not from their bucket).
_planner_seen: dict[tuple, object] = {}
_identity: dict[int, dict] = {}
_BASELINE = "planner"


def _device_identity(device) -> dict:
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _identity:
        props = torch.cuda.get_device_properties(index)
        # (not the marketing name: it reads empty where the ids table is not found, e.g.
        # under a profiler's preloaded runtime, which would hide every cached decision)
        _identity[index] = {
            "architecture": getattr(props, "gcnArchName", ""),
            "memory_bytes": props.total_memory,
            "compute_units": props.multi_processor_count,
            "library": _lib.lib().mt_source_digest().decode(),
            "tuner_source": hashlib.sha256(Path(__file__).read_bytes()).hexdigest(),
        }
    return _identity[index]


def _persistent_key(device, op, shape: dict, candidates) -> str:
    identity = _device_identity(device)
    context = (sorted(identity.items()), [astuple(c) for c in candidates], TUNER_VERSION,
               SWITCH_MARGIN, TIE_TOLERANCE, TAIL_QUANTILE, COLD_BYTES)
    return decision_key(op, shape, context)


def _read_entry(key):
    if not disk_cache_enabled():
        return None
    entry = load_decisions().get(key)
    return entry if isinstance(entry, dict) and "plan" in entry else None


def _read_decision(key, plan_type):
    """(found, plan): ``plan`` is None when the planner's plan was kept."""
    entry = _read_entry(key)
    if entry is None:
        return False, None
    if entry["plan"] is None:
        return True, None
    try:
        return True, plan_type(**entry["plan"])
    except TypeError:
        return False, None


def _write_decision(key, plan, record) -> None:
    if disk_cache_enabled():
        append_decision(key, {"plan": None if plan is None else asdict(plan), **record})


def cached_decisions() -> list:
    """Every decision in the log (the entries, newest per key)."""
    return [e for e in load_decisions().values() if isinstance(e, dict)]


def _tensor_bytes(*tensors) -> int:
    return sum(t.numel() * t.element_size() for t in tensors)


def _copies(weight_bytes: int) -> int:
    return max(2, min(MAX_COPIES, -(-COLD_BYTES // max(weight_bytes, 1))))


class _Bench:
    """Times dispatches replayed from HIP graphs on one side stream; owns its workspace (grown
    before any capture, so every graph keeps a valid pointer)."""

    def __init__(self, device, workspace_bytes):
        self.device = device
        self.ws = torch.zeros(max(workspace_bytes, 1 << 16), dtype=torch.uint8, device=device)
        self.stream = torch.cuda.Stream(device)
        # inputs, weight copies and the workspace were written on the caller's stream
        self.stream.wait_stream(torch.cuda.current_stream(device))
        self.graphs = []

    def capture(self, body):
        with torch.cuda.stream(self.stream):
            body()  # eager run first: the dispatch is checked outside capture
            self.stream.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.stream):
                body()
        self.graphs.append(g)
        return g

    def measure(self, graph):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(self.stream):
            start.record(self.stream)
            graph.replay()
            end.record(self.stream)
        end.synchronize()
        return start.elapsed_time(end) * 1e-3

    def close(self):
        self.graphs.clear()
        torch.cuda.synchronize(self.device)


def _tournament(bench, graphs, copies, cost, baseline=_BASELINE):
    """Seconds per dispatch of each key of ``graphs`` (``{key: graph}``), and the key chosen."""
    measure = bench.measure
    entries = list(graphs.items())
    for _, g in entries:  # one untimed replay each: clocks and caches in the steady state
        measure(g)
    provisional = {k: tail_quantile(v) for k, v in screen(entries, SCREEN_ROUNDS, measure).items()}
    best = min(provisional.values())
    alternatives = [k for k in provisional if k != baseline]
    fastest_alt = min(alternatives, key=provisional.__getitem__) if alternatives else None
    finalists = [(k, g) for k, g in entries
                 if provisional[k] <= best * FINALIST_SLACK or k in (baseline, fastest_alt)]
    timings = head_to_head(finalists, baseline, ABBA_BLOCKS, measure)
    timings = {k: t / copies for k, t in timings.items()}
    return timings, choose(timings, baseline, cost)


def _gate(result, reference, what):
    from .fidelity import affine_swiglu_compatible

    if not affine_swiglu_compatible(result, reference):
        raise RuntimeError(f"{what}: a plan failed the fidelity gate against the planner's plan")


def _tune_qmv_dispatch(values, weights, group_size, bits, layout):
    """Measure every plan of one dispatch shape (``values`` rows <= one dispatch) and return
    ``(plan or None, record)``."""
    plan, _, record = _tune_qmv_layouts(values, [(layout, weights)], group_size, bits)
    return plan, record


def _tune_qmv_layouts(values, weight_sets, group_size, bits):
    """Measure every plan of one dispatch shape over each ``(layout, weights)`` of
    ``weight_sets`` (the same weights in different code layouts; the first is the baseline's)
    and return ``(plan or None, layout, record)``: the fastest pair."""
    from .quantized import _as_u32

    L = _lib.lib()
    nproj = len(weight_sets[0][1]) // 3
    rows, k = values.shape
    dtype = values.dtype
    code = _dtype_code(dtype)
    sets = []
    for layout, weights in weight_sets:
        tensors = [_as_u32(t) if i % 3 == 0 else t.contiguous() for i, t in enumerate(weights)]
        sets.append((layout, tensors))
    layout0, tensors0 = sets[0]
    n = tensors0[0].shape[1] if layout0 == _LAYOUT_REPACKED else tensors0[0].shape[0]
    candidates = qmv_plan_candidates(rows, k, n, group_size, bits, nproj)
    copies = _copies(_tensor_bytes(*tensors0))
    rotations = {layout: [tensors] + [[t.clone() for t in tensors] for _ in range(copies - 1)]
                 for layout, tensors in sets}
    need = 0
    for plan in [None, *candidates]:
        install_qmv_plan(rows, k, n, group_size, bits, nproj, dtype, plan)
        need = max(need, L.mt_affine_qmv_workspace_bytes(rows, k, n, group_size, bits, nproj))
    install_qmv_plan(rows, k, n, group_size, bits, nproj, dtype, None)
    bench = _Bench(values.device, need)
    x = values.contiguous()
    outs = [torch.empty(rows, n, dtype=dtype, device=values.device) for _ in range(copies)]

    def body_for(layout):
        fn = ((L.mt_affine_qmv_repacked if layout == _LAYOUT_REPACKED else L.mt_affine_qmv)
              if nproj == 1 else
              (L.mt_affine_swiglu_repacked if layout == _LAYOUT_REPACKED
               else L.mt_affine_swiglu))

        def body():
            stream = torch.cuda.current_stream(values.device).cuda_stream
            for ts, out in zip(rotations[layout], outs):
                ptrs = [t.data_ptr() for t in ts]
                if nproj == 1:
                    args = (x.data_ptr(), *ptrs, None, out.data_ptr())
                else:
                    args = (x.data_ptr(), *ptrs, out.data_ptr())
                _lib.check(fn(*args, rows, k, n, group_size, bits, code, bench.ws.data_ptr(),
                              bench.ws.numel(), stream))

        return body

    baseline = (_BASELINE, layout0)
    graphs, reference = {}, None
    try:
        for layout, _ in sets:
            body = body_for(layout)
            for key, plan in [(_BASELINE, None), *[(c, c) for c in candidates]]:
                install_qmv_plan(rows, k, n, group_size, bits, nproj, dtype, plan)
                graphs[(key, layout)] = bench.capture(body)
                bench.stream.synchronize()
                if reference is None:
                    reference = outs[0].clone()
                else:
                    _gate(outs[0], reference, "affine plan tuning")
        install_qmv_plan(rows, k, n, group_size, bits, nproj, dtype, None)
        # cost: workgroups, then the baseline's layout
        timings, chosen = _tournament(
            bench, graphs, copies,
            lambda key: (-1 if key[0] == _BASELINE else key[0].workgroups, key[1] != layout0),
            baseline)
    finally:
        install_qmv_plan(rows, k, n, group_size, bits, nproj, dtype, None)
        bench.close()
    planner = qmv_plan(rows, k, n, group_size, bits, nproj, dtype)
    plan = None if chosen[0] == _BASELINE else chosen[0]
    record = {
        "planner": asdict(planner),
        "planner_us": round(timings[baseline] * 1e6, 3),
        "chosen_us": round(timings[chosen] * 1e6, 3),
        "copies": copies,
    }
    if len(sets) > 1:
        record["layout"] = _LAYOUT_NAMES[chosen[1]]
    return plan, chosen[1], record


def _qmv_shape(rows, k, n, group_size, bits, nproj, dtype) -> dict:
    return {"rows": row_bucket(rows), "input_features": k, "output_features": n,
            "group_size": group_size, "bits": bits, "nproj": nproj, "dtype": str(dtype)}


def dispatch_rows(rows: int, group_size: int) -> list[int]:
    """Rows of the dispatches a call of ``rows`` rows makes (32 at a time, 16 for groups of
    32), distinct buckets only."""
    chunk = 16 if group_size == 32 else 32
    out = []
    for r in (min(rows, chunk), rows % chunk if rows > chunk else 0):
        if r and row_bucket(r) not in {row_bucket(v) for v in out}:
            out.append(r)
    return out


def ensure_qmv_plans(values, weights, *, group_size, bits, autotune=True, retune=False):
    """Make the dispatches of ``values`` (any leading shape) over ``weights`` take their tuned
    plans: ``weights`` is ``(w, scales, biases)`` (QMV) or the gate triple then the up triple
    (SwiGLU), in MLX or repacked layout (measured in the layout given; the decision applies to
    both). Per dispatch shape: this process's decision, else the disk cache's, else
    (``autotune`` and tuning enabled, outside graph capture) a measurement, which is then
    cached. Returns ``{rows: plan or None}`` (None: the planner's plan)."""
    from .quantized import _repacked

    nproj = len(weights) // 3
    layout = _LAYOUT_REPACKED if _repacked(weights[0]) else _LAYOUT_MLX
    k = values.shape[-1]
    n = weights[0].shape[1] if layout == _LAYOUT_REPACKED else weights[0].shape[0]
    x = values.reshape(-1, k)
    out = {}
    with _lock:
        for rows in dispatch_rows(x.shape[0], group_size):
            mem = ("qmv", values.device.index, row_bucket(rows), k, n, group_size, bits, nproj,
                   values.dtype)
            if mem in _decided and not retune:
                out[rows] = _decided[mem]
                continue
            candidates = qmv_plan_candidates(rows, k, n, group_size, bits, nproj)
            shape = _qmv_shape(rows, k, n, group_size, bits, nproj, values.dtype)
            key = _persistent_key(values.device, "affine_qmv", shape, candidates)
            found, plan = (False, None) if retune else _read_decision(key, QmvPlan)
            if not found:
                if (not autotune or not tuning_enabled()
                        or torch.cuda.is_current_stream_capturing()):
                    out[rows] = None
                    _resolved.setdefault(mem, "planner")
                    _planner_seen.setdefault(
                        mem, qmv_plan(rows, k, n, group_size, bits, nproj, values.dtype))
                    continue  # not decided: the planner's plan, and measure another time
                plan, record = _tune_qmv_dispatch(x[:rows], weights, group_size, bits, layout)
                _write_decision(key, plan, {"op": "affine_qmv", **shape, **record})
            install_qmv_plan(rows, k, n, group_size, bits, nproj, values.dtype, plan)
            _decided[mem] = plan
            _resolved[mem] = "cached" if found else "measured"
            out[rows] = plan
    return out


_LAYOUT_CODES = {name: code for code, name in _LAYOUT_NAMES.items()}


def ensure_qmv_layout(values, layouts, *, group_size, bits, autotune=True, retune=False):
    """``ensure_qmv_plans`` over one weight held in several code layouts: ``layouts`` maps
    ``"repacked"`` and/or ``"mlx"`` to the weights (as for ``ensure_qmv_plans``) in that layout,
    the first being the default (its planner plan is the baseline). The first dispatch shape's
    plans are measured over every layout, which picks the plan and the layout together (plans
    are layout-free: results are bit-identical in either layout); the other dispatch shapes are
    then tuned in that layout. Returns the name of the layout to keep: the first when nothing
    was measured (tuning off, or inside graph capture, with no cached decision)."""
    names = list(layouts)
    if not names or any(name not in _LAYOUT_CODES for name in names):
        raise ValueError('layouts must map "repacked" and/or "mlx" to weights')
    if len(names) == 1:
        ensure_qmv_plans(values, layouts[names[0]], group_size=group_size, bits=bits,
                         autotune=autotune, retune=retune)
        return names[0]
    from .quantized import _repacked

    for name in names:
        if _repacked(layouts[name][0]) != (name == "repacked"):
            raise ValueError(f"the {name!r} weights are not in that layout")
    first = layouts[names[0]]
    nproj = len(first) // 3
    k = values.shape[-1]
    n = first[0].shape[1] if names[0] == "repacked" else first[0].shape[0]
    x = values.reshape(-1, k)
    rows = dispatch_rows(x.shape[0], group_size)[0]
    chosen = names[0]
    with _lock:
        mem = ("qmv", values.device.index, row_bucket(rows), k, n, group_size, bits, nproj,
               values.dtype)
        lmem = (*mem, tuple(names))
        if lmem in _decided_layouts and not retune:
            plan, chosen = _decided_layouts[lmem]
        else:
            candidates = qmv_plan_candidates(rows, k, n, group_size, bits, nproj)
            shape = _qmv_shape(rows, k, n, group_size, bits, nproj, values.dtype)
            key = _persistent_key(values.device, "affine_qmv_layout",
                                  {**shape, "layouts": names}, candidates)
            found, plan, cached = (False, None, None) if retune else _read_layout_decision(key)
            decided = found and cached in names
            if decided:
                chosen = cached
                _resolved[mem] = "cached"
            elif autotune and tuning_enabled() and not torch.cuda.is_current_stream_capturing():
                plan, code, record = _tune_qmv_layouts(
                    x[:rows], [(_LAYOUT_CODES[name], layouts[name]) for name in names],
                    group_size, bits)
                chosen = _LAYOUT_NAMES[code]
                _write_decision(key, plan, {"op": "affine_qmv_layout", **shape,
                                            "layouts": names, **record})
                decided = True
                _resolved[mem] = "measured"
            if decided:
                install_qmv_plan(rows, k, n, group_size, bits, nproj, values.dtype, plan)
                _decided[mem] = plan
                _decided_layouts[lmem] = (plan, chosen)
    ensure_qmv_plans(values, layouts[chosen], group_size=group_size, bits=bits,
                     autotune=autotune, retune=False)
    return chosen


def _read_layout_decision(key):
    """(found, plan, layout name) of a cached layout decision."""
    found, plan = _read_decision(key, QmvPlan)
    if not found:
        return False, None, None
    entry = _read_entry(key) or {}
    return True, plan, entry.get("layout")


def _tune_gemm(values, weight, scales, biases, group_size):
    L = _lib.lib()
    from .quantized import _as_u32

    rows, k = values.shape
    w, s, b = _as_u32(weight), scales.contiguous(), biases.contiguous()
    n = w.shape[0]
    dtype = values.dtype
    code = _dtype_code(dtype)
    candidates = gemm_plan_candidates(rows, k, n, group_size)
    copies = _copies(_tensor_bytes(w, s, b))
    rotation = [(w, s, b)] + [(w.clone(), s.clone(), b.clone()) for _ in range(copies - 1)]
    need = 0
    for plan in [None, *candidates]:
        install_gemm_plan(rows, k, n, group_size, dtype, plan)
        need = max(need, L.mt_affine_gemm_workspace_bytes(rows, k, n, group_size, 4))
    install_gemm_plan(rows, k, n, group_size, dtype, None)
    bench = _Bench(values.device, need)
    x = values.contiguous()
    outs = [torch.empty(rows, n, dtype=dtype, device=values.device) for _ in range(copies)]

    def body():
        stream = torch.cuda.current_stream(values.device).cuda_stream
        for (ww, ss, bb), out in zip(rotation, outs):
            _lib.check(L.mt_affine_gemm(x.data_ptr(), ww.data_ptr(), ss.data_ptr(), bb.data_ptr(),
                                        out.data_ptr(), rows, k, n, group_size, 4, code,
                                        bench.ws.data_ptr(), bench.ws.numel(), stream))

    graphs, reference = {}, None
    try:
        for key, plan in [(_BASELINE, None), *[(c, c) for c in candidates]]:
            install_gemm_plan(rows, k, n, group_size, dtype, plan)
            graphs[key] = bench.capture(body)
            bench.stream.synchronize()
            if reference is None:
                reference = outs[0].clone()
            else:
                _gate(outs[0], reference, "affine matmul plan tuning")
        install_gemm_plan(rows, k, n, group_size, dtype, None)
        timings, chosen = _tournament(
            bench, graphs, copies,
            lambda key: -1 if key == _BASELINE else key.workgroups(rows, n))
    finally:
        install_gemm_plan(rows, k, n, group_size, dtype, None)
        bench.close()
    planner = gemm_plan(rows, k, n, group_size, dtype)
    plan = None if chosen == _BASELINE else chosen
    return plan, {"planner": asdict(planner), "planner_us": round(timings[_BASELINE] * 1e6, 3),
                  "chosen_us": round(timings[chosen] * 1e6, 3), "copies": copies}


def ensure_gemm_plan(values, weight, scales, biases, *, group_size, autotune=True, retune=False):
    """``ensure_qmv_plans`` for the prefill GEMM (4-bit codes in MLX layout)."""
    k = values.shape[-1]
    x = values.reshape(-1, k)
    rows = x.shape[0]
    n = weight.shape[0]
    with _lock:
        mem = ("gemm", values.device.index, row_bucket(rows), k, n, group_size, values.dtype)
        if mem in _decided and not retune:
            return _decided[mem]
        candidates = gemm_plan_candidates(rows, k, n, group_size)
        shape = {"rows": row_bucket(rows), "input_features": k, "output_features": n,
                 "group_size": group_size, "bits": 4, "dtype": str(values.dtype)}
        key = _persistent_key(values.device, "affine_matmul", shape, candidates)
        found, plan = (False, None) if retune else _read_decision(key, GemmPlan)
        if not found:
            if not autotune or not tuning_enabled() or torch.cuda.is_current_stream_capturing():
                _resolved.setdefault(mem, "planner")
                return None
            plan, record = _tune_gemm(x, weight, scales, biases, group_size)
            _write_decision(key, plan, {"op": "affine_matmul", **shape, **record})
        install_gemm_plan(rows, k, n, group_size, values.dtype, plan)
        _decided[mem] = plan
        _resolved[mem] = "cached" if found else "measured"
        return plan


# Row counts a dense plan is timed at: one plan serves every row count (the per-row bit
# identity), so each candidate's graph holds one dispatch at each of them and is scored on the sum.
DENSE_TUNING_ROWS = (1, 16, 128)


def _tune_dense(weights, dtype):
    L = _lib.lib()
    nproj = len(weights)
    n, k = weights[0].shape
    device = weights[0].device
    candidates = dense_plan_candidates(k, n, nproj)
    copies = _copies(_tensor_bytes(*weights))
    rotation = [tuple(weights)] + [tuple(w.clone() for w in weights) for _ in range(copies - 1)]
    need = 0
    for plan in [None, *candidates]:
        install_dense_plan(k, n, nproj, dtype, plan)
        need = max(need, L.mt_dense_workspace_bytes(max(DENSE_TUNING_ROWS), k, n, nproj))
    install_dense_plan(k, n, nproj, dtype, None)
    bench = _Bench(device, need)
    gen = torch.Generator(device=device)
    gen.manual_seed(0)
    xs = [torch.randn(m, k, generator=gen, device=device).to(dtype) for m in DENSE_TUNING_ROWS]
    res = [torch.randn(m, n, generator=gen, device=device).to(dtype) for m in DENSE_TUNING_ROWS]
    outs = [torch.empty(m, n, dtype=dtype, device=device) for m in DENSE_TUNING_ROWS]
    code = _dtype_code(dtype)

    def body():
        stream = torch.cuda.current_stream(device).cuda_stream
        for x, r, out in zip(xs, res, outs):
            for ws in rotation:
                if nproj == 2:
                    _lib.check(L.mt_dense_swiglu(x.data_ptr(), ws[0].data_ptr(), ws[1].data_ptr(),
                                                 out.data_ptr(), x.shape[0], k, n, code,
                                                 bench.ws.data_ptr(), bench.ws.numel(), stream))
                else:
                    _lib.check(L.mt_dense_residual_qmv(
                        x.data_ptr(), ws[0].data_ptr(), r.data_ptr(), out.data_ptr(), x.shape[0],
                        k, n, code, bench.ws.data_ptr(), bench.ws.numel(), stream))

    graphs, reference = {}, None
    try:
        for key, plan in [(_BASELINE, None), *[(c, c) for c in candidates]]:
            install_dense_plan(k, n, nproj, dtype, plan)
            graphs[key] = bench.capture(body)
            bench.stream.synchronize()
            if reference is None:
                reference = outs[-1].clone()
            else:
                _gate(outs[-1], reference, "dense plan tuning")
        install_dense_plan(k, n, nproj, dtype, None)
        timings, chosen = _tournament(bench, graphs, copies,
                                      lambda key: -1 if key == _BASELINE else key.workgroups(n))
    finally:
        install_dense_plan(k, n, nproj, dtype, None)
        bench.close()
    planner = dense_plan(k, n, nproj, dtype)
    plan = None if chosen == _BASELINE else chosen
    return plan, {"planner": asdict(planner), "planner_us": round(timings[_BASELINE] * 1e6, 3),
                  "chosen_us": round(timings[chosen] * 1e6, 3), "copies": copies,
                  "rows_timed": list(DENSE_TUNING_ROWS)}


def ensure_dense_plan(weights, dtype, *, autotune=True, retune=False):
    """The dense plan of a shape (``weights``: the ``[N, K]`` gate and up matrices, or one
    projection's), measured once per process and persisted like the affine decisions. The
    decision is keyed by (K, N, projections, dtype) only and installed for every row count, so
    that each output row stays bit-identical to that row run alone. Returns the plan (None:
    the planner's)."""
    nproj = len(weights)
    n, k = weights[0].shape
    device = weights[0].device
    with _lock:
        mem = ("dense", device.index, k, n, nproj, dtype)
        if mem in _decided and not retune:
            return _decided[mem]
        candidates = dense_plan_candidates(k, n, nproj)
        shape = {"input_features": k, "output_features": n, "projections": nproj,
                 "dtype": str(dtype), "rows_timed": list(DENSE_TUNING_ROWS)}
        key = _persistent_key(device, "dense", shape, candidates)
        found, plan = (False, None) if retune else _read_decision(key, DensePlan)
        if not found:
            if not autotune or not tuning_enabled() or torch.cuda.is_current_stream_capturing():
                _resolved.setdefault(mem, "planner")
                return None
            plan, record = _tune_dense([w.contiguous() for w in weights], dtype)
            _write_decision(key, plan, {"op": "dense", **shape, **record})
        install_dense_plan(k, n, nproj, dtype, plan)
        _decided[mem] = plan
        _resolved[mem] = "cached" if found else "measured"
        return plan


def dispatches(op: str) -> tuple:
    """This process's dispatch decisions for one operation, as the reference's
    ``mlx_affine_swiglu_dispatches`` / ``mlx_affine_residual_qmv_dispatches`` /
    ``mlx_affine_matmul_dispatches`` report theirs (``metile/backends/mlx_quantized.py:1627,1835``;
    ``metile/backends/mlx_affine.py:409``): one dict per dispatch shape resolved so far, sorted
    by shape. ``op`` is ``"swiglu"`` (two projections), ``"qmv"`` (one projection, with or
    without a residual: the plan does not depend on it) or ``"matmul"`` (the prefill GEMM).

    Each dict holds the shape (``rows`` is the row bucket the decision covers), the plan the
    library runs for it now, the code layout when a layout decision picked one, and
    ``source``: ``"measured"``, ``"cached"`` (from the decision cache on disk) or ``"planner"``
    (nothing decided; the library's own plan)."""
    if op not in ("swiglu", "qmv", "matmul"):
        raise ValueError('op must be "swiglu", "qmv" or "matmul"')
    with _lock:
        resolved = dict(_resolved)
        decided = dict(_decided)
        layouts = dict(_decided_layouts)
        seen = dict(_planner_seen)
    out = []
    for mem, source in resolved.items():
        if op == "matmul":
            if mem[0] != "gemm":
                continue
            _, device, bucket, k, n, group_size, dtype = mem
            plan = decided.get(mem) or gemm_plan(bucket, k, n, group_size, dtype)
            out.append({"rows": bucket, "input_features": k, "output_features": n,
                        "dtype": str(dtype), "group_size": group_size, "bits": 4,
                        "device": device, "kernel": plan.kernel, "tile_m": plan.tile_m,
                        "tile_n": plan.tile_n, "ksplit": plan.ksplit, "order": plan.order,
                        "source": source})
            continue
        if mem[0] != "qmv" or mem[7] != (2 if op == "swiglu" else 1):
            continue
        _, device, bucket, k, n, group_size, bits, nproj, dtype = mem
        plan = (decided.get(mem) or seen.get(mem)
                or qmv_plan(bucket, k, n, group_size, bits, nproj, dtype))
        layout = next((chosen for key, (_p, chosen) in layouts.items() if key[:9] == mem), None)
        out.append({"rows": bucket, "input_features": k, "output_features": n,
                    "dtype": str(dtype), "group_size": group_size, "bits": bits,
                    "device": device, "kernel": plan.kernel, "ksplit": plan.ksplit,
                    "strips": plan.strips, "tiles": plan.tiles, "order": plan.order,
                    "layout": layout, "source": source})
    out.sort(key=lambda d: (d["device"], d["input_features"], d["output_features"], d["dtype"],
                            d["group_size"], d["bits"], d["rows"]))
    return tuple(out)
