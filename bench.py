"""Benchmark of the quantized-projection hot path on one MI355X.

Headline workload: the INT4 fused SwiGLU MLP at Qwen2.5-1.5B shape (hidden
1536, intermediate 8960, group 64, bf16 activations) over a stack of 28 distinct layers
(650 MB of packed weights, 2.5x the 256 MB Infinity Cache), so every step streams its weights
from HBM. A step is one pass of the hot path over one batch: the M=1 decode row through all 28
layer MLPs (fused gate/up SwiGLU kernel, then the down projection with the residual epilogue),
replayed from a HIP graph whose outputs are first checked bit-for-bit against an eager run.
Weights are seeded synthetic data of the BASELINE recipe (codes uniform in 0..15,
scale = |N(0,1)|*0.02 in bf16, bias = -8*scale), generated in MLX's layout. Each stage's
weights are kept in the code layout its tuned M=1 plan reads fastest, decided with the plans
ahead of time and outside every timed region (``metile_amd.tuning.ensure_qmv_layout``, as the
library's executors do when they bind; ``layouts`` in the JSON line): the step-major repack of
``affine_repack`` or MLX's rows (the reference's executors likewise choose between their
repacked and plain schedules). The results are bit-identical in either layout; all-MLX codes are
also timed at M=1 (``native_layout``).

``value`` is the whole-job algorithmic HBM throughput of the M=1 step: packed weights, scales,
biases, activations in and out. The JSON line also carries:
* ``rows``: the same MLP at M = 1, 2, 4, 8, 16, 32 (us per layer call, GB/s);
* ``roofline``: the dominant kernel (the fused SwiGLU at M=1), timed alone with HIP events on
  the stream it runs on;
* ``configs``: the other BASELINE configs (0: one INT4 projection 1536->8960 at M=1..32;
  2: dense BF16 MLP at Llama-3.2-1B shape; 3: INT8 projection 5120->17408; 4: INT4 prefill
  GEMM at M=512), each over enough distinct weight copies to defeat the Infinity Cache;
* ``ceiling``: the measured streaming-read rate of one launch at the same byte counts;
* ``cpu_baseline``: the NumPy oracle on this host's cores.

Every shape first takes its tuned plan (``metile_amd.tuning``, untimed, before the timed
region; ``tuning`` in the JSON line lists each decision with the planner's and the chosen plan's
time); ``--no-tune`` keeps the planner's plans.

Usage: ``python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-tune]``.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

HIDDEN, INTER, GROUP, BITS, LAYERS = 1536, 8960, 64, 4, 28
ROWS = (1, 2, 4, 8, 16, 32)
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
STACK_BYTES = 600 << 20  # distinct weight bytes per timed rotation (> 2x the 256 MB MALL)


def proj_weight_bytes(k, n, bits=BITS, group=GROUP):
    return n * k * bits // 8 + 2 * 2 * n * (k // group)


def mlp_bytes(m):
    """Algorithmic bytes of one layer MLP call at m rows: gate+up+down packed weights, scales
    and biases, x in, residual in, y out, and the hidden activation's store and reload."""
    w = 2 * proj_weight_bytes(HIDDEN, INTER) + proj_weight_bytes(INTER, HIDDEN)
    act = 2 * m * HIDDEN * 3 + 2 * 2 * m * INTER
    return w + act


def make_affine(gen, device, k, n, bits=BITS, group=GROUP):
    words = torch.randint(-2**31, 2**31, (n, k * bits // 32), generator=gen, device=device,
                          dtype=torch.int64).to(torch.int32)
    coef, zero = (0.02, 8.0) if bits == 4 else (0.002, 128.0)
    s = (torch.randn(n, k // group, generator=gen, device=device).abs() * coef).to(torch.bfloat16)
    b = (s.float() * -zero).to(torch.bfloat16)
    return words, s, b


def make_layer(gen, device):
    return (make_affine(gen, device, HIDDEN, INTER), make_affine(gen, device, HIDDEN, INTER),
            make_affine(gen, device, INTER, HIDDEN))


def repacked(mt, triple, bits=BITS):
    """The (weight, scales, biases) triple with its codes repacked step-major (one-time)."""
    w, s, b = triple
    return mt.affine_repack(w, bits=bits), s, b


# Untimed replays continue for at least this long before timing starts: the first replays after
# an idle host phase (allocation, capture, tuning) ran up to 18% slower (prefill down GEMM:
# 57.2 us on the first graph of a shape, 48.7 us once clocks had settled).
MIN_WARM_MS = 25.0


def time_graph(graph, stream, steps, warmup):
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < MIN_WARM_MS:
        for _ in range(max(warmup, 1)):
            graph.replay()
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per replay


def capture(fn, stream):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    return g


def timed(fn, stream, steps, warmup, calls):
    """Run ``fn`` eagerly (allocates workspaces outside capture), capture it, check that a
    replay reproduces the eager outputs bit for bit, and return us per call."""
    outs = fn()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    holder = {}

    def body():
        holder["outs"] = fn()

    graph = capture(body, stream)
    graph.replay()
    torch.cuda.synchronize()
    for a, b in zip(eager, holder["outs"]):
        if not torch.equal(a.view(torch.int16), b.view(torch.int16)):
            raise RuntimeError("graph replay differs from the eager run")
    return time_graph(graph, stream, steps, warmup) * 1e3 / calls


def copies_for(nbytes):
    return max(2, -(-STACK_BYTES // nbytes))


def tune(args, values, weights, bits=BITS):
    """The plans this shape's dispatches take (untimed, before the timed region): the tuner's
    decision (``metile_amd.tuning``: every plan the library lists, timed from HIP graphs over
    cold weights), as the reference's tuned entries and executors do on first use."""
    if args.no_tune:
        return
    from metile_amd import tuning

    tuning.ensure_qmv_plans(values, weights, group_size=GROUP, bits=bits)


def choose_layout(args, values, native, packed, bits=BITS):
    """The code layout one projection's weights are kept in (untimed, before the timed region):
    the tuner times every plan over both layouts (``metile_amd.tuning.ensure_qmv_layout``) and
    keeps the faster pair, as the library's executors do when they bind; ``--no-tune`` keeps
    the repacked codes. ``native``/``packed``: the weights as for ``tune``, in MLX's layout and
    repacked."""
    if args.no_tune:
        return "repacked"
    from metile_amd import tuning

    return tuning.ensure_qmv_layout(values, {"repacked": packed, "mlx": native},
                                    group_size=GROUP, bits=bits)


# ---- sections ---------------------------------------------------------------------------------


def make_stack(mt, gen, device):
    """The 28-layer stack in MLX's layout and repacked step-major (``affine_repack``)."""
    native = [make_layer(gen, device) for _ in range(LAYERS)]
    packed = [tuple(repacked(mt, t) for t in layer) for layer in native]
    torch.cuda.synchronize()
    return native, packed


def stack_layers(args, gen, device, native, packed, m):
    """The stack as a caller serving ``m`` rows keeps it: each stage's weights in the layout its
    plan at ``m`` rows reads fastest (``choose_layout``). Returns ``(layers, layouts)``."""
    (ng, nu, nd), (pg, pu, pd) = native[0], packed[0]
    x = torch.randn(m, HIDDEN, generator=gen, device=device).to(torch.bfloat16)
    up_layout = choose_layout(args, x, (*ng, *nu), (*pg, *pu))
    from metile_amd import quantized as Q

    h = Q.affine_swiglu(x, *(pg if up_layout == "repacked" else ng),
                        *(pu if up_layout == "repacked" else nu), group_size=GROUP, bits=BITS)
    down_layout = choose_layout(args, h, nd, pd)
    layers = [((p if up_layout == "repacked" else n)[0], (p if up_layout == "repacked" else n)[1],
               (p if down_layout == "repacked" else n)[2]) for n, p in zip(native, packed)]
    return layers, {"gate_up": up_layout, "down": down_layout}


def kernel_label(k, n, nproj):
    """The kernel instance an M=1 dispatch of this shape runs under the plan installed now."""
    from metile_amd import tuning

    plan = tuning.qmv_plan(1, k, n, GROUP, BITS, nproj, torch.bfloat16)
    if plan.kernel == "gemv":
        waves, chunks = plan.tiles, k * BITS // 128
        one_pass = chunks <= 64 * waves
        groups = 64 * waves // chunks if one_pass and chunks % 16 == 0 else 1
        cols = n // plan.strips // groups
        flags = f"{str(one_pass).lower()}, {str(groups > 1).lower()}"
        return (f"affine_gemv_kernel<{BITS}, 0, 1, {nproj}, {cols}, {flags}> "
                f"({plan.strips} workgroups of {waves} waves, {groups} column groups each)")
    if plan.kernel == "staged":
        return (f"affine_qmv_lds_kernel<{BITS}, 0, 8, {nproj}, ...> "
                f"({plan.strips} strips, {plan.ksplit} K splits)")
    return f"affine_qmv_kernel<{BITS}, 0, ..., {nproj}, ...> ({plan.ksplit} K splits)"


def section_mlp(mt, gen, device, stream, args):
    native, packed = make_stack(mt, gen, device)
    kernel = {}
    wbytes = 2 * proj_weight_bytes(HIDDEN, INTER) + proj_weight_bytes(INTER, HIDDEN)
    rows_out, step_ms = {}, None
    rows = sorted({1, *(int(v) for v in args.rows.split(","))})
    for m in rows:
        layers, layouts = stack_layers(args, gen, device, native, packed, m)
        if m == 1:
            kernel["layouts"] = layouts
        x = torch.randn(m, HIDDEN, generator=gen, device=device).to(torch.bfloat16)
        res = torch.randn(m, HIDDEN, generator=gen, device=device).to(torch.bfloat16)

        def stack():
            return [mt.affine_mlp(x, g, u, d, group_size=GROUP, bits=BITS, residual=res)
                    for (g, u, d) in layers]

        g0, u0, d0 = layers[0]
        tune(args, x, (*g0, *u0))
        tune(args, torch.randn(m, INTER, generator=gen, device=device).to(torch.bfloat16), d0)
        steps = args.steps if m == 1 else max(10, args.steps // 4)
        us = timed(stack, stream, steps, args.warmup, LAYERS)
        rows_out[str(m)] = {
            "layouts": layouts,
            "us_per_mlp_call": round(us, 3),
            "hbm_GBps": round(mlp_bytes(m) / us / 1e3, 1),
            "weight_GBps": round(wbytes / us / 1e3, 1),
            "frac_of_peak": round(mlp_bytes(m) / us / 1e3 / HBM_PEAK_GBS, 4),
        }
        if m == 1:
            step_ms = us * LAYERS / 1e3
            hs = [torch.randn(m, INTER, generator=gen, device=device).to(torch.bfloat16)
                  for _ in range(LAYERS)]

            def swiglu():
                return [mt.affine_swiglu(x, *g, *u, group_size=GROUP, bits=BITS)
                        for (g, u, _d) in layers]

            def down():
                return [mt.affine_qmv(h, *d, group_size=GROUP, bits=BITS, residual=res)
                        for h, (_g, _u, d) in zip(hs, layers)]

            kernel["swiglu_label"] = kernel_label(HIDDEN, INTER, 2)
            kernel["down_label"] = kernel_label(INTER, HIDDEN, 1)
            kernel["swiglu_us"] = timed(swiglu, stream, args.steps, args.warmup, LAYERS)
            kernel["down_us"] = timed(down, stream, args.steps, args.warmup, LAYERS)
            kernel["swiglu_bytes"] = (2 * proj_weight_bytes(HIDDEN, INTER) + 2 * m * HIDDEN
                                      + 2 * m * INTER)
            kernel["down_bytes"] = proj_weight_bytes(INTER, HIDDEN) + 2 * m * INTER + 4 * m * HIDDEN

            def native_stack():
                return [mt.affine_mlp(x, g, u, d, group_size=GROUP, bits=BITS, residual=res)
                        for (g, u, d) in native]

            def native_swiglu():
                return [mt.affine_swiglu(x, *g, *u, group_size=GROUP, bits=BITS)
                        for (g, u, _d) in native]

            def native_down():
                return [mt.affine_qmv(h, *d, group_size=GROUP, bits=BITS, residual=res)
                        for h, (_g, _u, d) in zip(hs, native)]

            nus = timed(native_stack, stream, steps, args.warmup, LAYERS)
            kernel["native_layout"] = {
                "us_per_mlp_call": round(nus, 3),
                "hbm_GBps": round(mlp_bytes(m) / nus / 1e3, 1),
                "swiglu_us": round(timed(native_swiglu, stream, args.steps, args.warmup,
                                         LAYERS), 3),
                "down_us": round(timed(native_down, stream, args.steps, args.warmup, LAYERS), 3),
            }
    del layers, native
    return rows_out, kernel, step_ms


def section_qmv(mt, gen, device, stream, args, k, n, bits, rows):
    """One affine projection over a rotation of distinct copies (configs 0 and 3); at each row
    count the codes are in the layout the tuner picks for it (both are held)."""
    wb = proj_weight_bytes(k, n, bits)
    copies = copies_for(wb)
    native = [make_affine(gen, device, k, n, bits) for _ in range(copies)]
    packed = [repacked(mt, w, bits) for w in native]
    out = {}
    for m in rows:
        x = torch.randn(m, k, generator=gen, device=device).to(torch.bfloat16)
        layout = choose_layout(args, x, native[0], packed[0], bits)
        ws = packed if layout == "repacked" else native
        us = timed(lambda: [mt.affine_qmv(x, *w, group_size=GROUP, bits=bits) for w in ws],
                   stream, max(10, args.steps // 4), args.warmup, copies)
        total = wb + 2 * m * k + 2 * m * n
        out[str(m)] = {"layout": layout, "us": round(us, 3),
                       "hbm_GBps": round(total / us / 1e3, 1),
                       "frac_of_peak": round(total / us / 1e3 / HBM_PEAK_GBS, 4)}
    del native, packed
    return {"K": k, "N": n, "bits": bits, "group_size": GROUP, "copies": copies,
            "bytes_per_call_M1": wb + 2 * k + 2 * n, "rows": out}


def section_dense(mt, gen, device, stream, args):
    """Dense BF16 SwiGLU MLP at Llama-3.2-1B shape (config 2)."""
    h, i = 2048, 8192
    wbytes = 3 * 2 * h * i
    copies = copies_for(wbytes)
    ws = [tuple((torch.randn(n, k, generator=gen, device=device) * 0.02).to(torch.bfloat16)
                for n, k in ((i, h), (i, h), (h, i))) for _ in range(copies)]
    out = {}
    for m in (1, 2, 8, 16, 32, 128):
        x = torch.randn(m, h, generator=gen, device=device).to(torch.bfloat16)
        res = torch.randn(m, h, generator=gen, device=device).to(torch.bfloat16)

        def stack():
            return [mt.dense_qmv(mt.dense_swiglu(x, g, u), d, res) for (g, u, d) in ws]

        us = timed(stack, stream, max(10, args.steps // 4), args.warmup, copies)
        total = wbytes + 2 * m * h * 3 + 4 * m * i
        out[str(m)] = {"us_per_mlp_call": round(us, 3), "hbm_GBps": round(total / us / 1e3, 1),
                       "weight_GBps": round(wbytes / us / 1e3, 1),
                       "frac_of_peak": round(total / us / 1e3 / HBM_PEAK_GBS, 4)}
    del ws
    return {"hidden": h, "intermediate": i, "copies": copies, "rows": out}


def section_prefill(mt, gen, device, stream, args):
    """INT4 prefill GEMM at M=512, Qwen2.5-1.5B up and down shapes (config 4)."""
    out = {}
    for name, k, n in (("up", HIDDEN, INTER), ("down", INTER, HIDDEN)):
        copies = copies_for(proj_weight_bytes(k, n))
        ws = [make_affine(gen, device, k, n) for _ in range(copies)]
        x = torch.randn(512, k, generator=gen, device=device).to(torch.bfloat16)
        if not args.no_tune:
            from metile_amd import tuning

            tuning.ensure_gemm_plan(x, *ws[0], group_size=GROUP)
        us = timed(lambda: [mt.affine_matmul(x, *w, group_size=GROUP, bits=BITS) for w in ws],
                   stream, max(10, args.steps // 4), args.warmup, copies)
        flops = 2 * 512 * k * n
        out[name] = {"K": k, "N": n, "M": 512, "copies": copies, "us": round(us, 3),
                     "TFLOPs": round(flops / us / 1e6, 1),
                     "frac_of_mfma_peak": round(flops / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4)}
        del ws
    return out


def section_ceiling(mt, device, stream, args):
    """Streaming-read rate of one launch over distinct buffers of each byte count."""
    from metile_amd import _lib

    lib = _lib.lib()
    sink = torch.empty(65536, dtype=torch.int32, device=device)
    out = {}
    for label, nbytes in (("7.7MB", 7_762_432), ("15.5MB", 15_503_872), ("23.2MB", 23_224_320),
                          ("100.7MB", 100_663_296)):
        copies = copies_for(nbytes)
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=device) for _ in range(copies)]
        for b in bufs:
            b.fill_(1)
        best = None
        for blocks in (256, 512, 1024):
            def run():
                for b in bufs:
                    _lib.check(lib.mt_stream_read(b.data_ptr(), nbytes, sink.data_ptr(), blocks,
                                                  torch.cuda.current_stream(device).cuda_stream))
                return [sink]

            with torch.cuda.stream(stream):
                run()
                torch.cuda.synchronize()
                g = capture(run, stream)
                us = time_graph(g, stream, max(10, args.steps // 4), args.warmup) * 1e3 / copies
            if best is None or us < best[0]:
                best = (us, blocks)
        out[label] = {"us": round(best[0], 3), "GBps": round(nbytes / best[0] / 1e3, 1),
                      "blocks": best[1]}
        del bufs
    return out


def traffic_probe(mt, gen, device, args):
    """Eager launches for the HBM-traffic counter runs (rocprofv3 --pmc FETCH_SIZE, then
    WRITE_SIZE): a plain 256 MiB device copy (the calibration kernel of known size), then the
    headline SwiGLU and down kernels over the 28-layer stack (layouts and plans as benchmarked:
    run with the decision cache of a tuned run and METILE_AMD_DISABLE_TUNING=1, so that no
    candidate plan is measured here), three passes each."""
    src = torch.empty(256 << 20, dtype=torch.uint8, device=device).fill_(3)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    native, packed = make_stack(mt, gen, device)
    layers, layouts = stack_layers(args, gen, device, native, packed, 1)
    x = torch.randn(1, HIDDEN, generator=gen, device=device).to(torch.bfloat16)
    res = torch.randn(1, HIDDEN, generator=gen, device=device).to(torch.bfloat16)
    hs = [torch.randn(1, INTER, generator=gen, device=device).to(torch.bfloat16)
          for _ in range(LAYERS)]
    for _ in range(3):
        for g, u, _d in layers:
            mt.affine_swiglu(x, *g, *u, group_size=GROUP, bits=BITS)
        for h, (_g, _u, d) in zip(hs, layers):
            mt.affine_qmv(h, *d, group_size=GROUP, bits=BITS, residual=res)
    torch.cuda.synchronize()
    print(json.dumps({"traffic_probe": "done", "copy_bytes": 256 << 20, "layouts": layouts}),
          flush=True)


def prefill_probe(mt, gen, device):
    """Eager launches for the prefill GEMM counter runs: three of each config-4 projection."""
    for k, n in ((HIDDEN, INTER), (INTER, HIDDEN)):
        w = make_affine(gen, device, k, n)
        x = torch.randn(512, k, generator=gen, device=device).to(torch.bfloat16)
        for _ in range(3):
            mt.affine_matmul(x, *w, group_size=GROUP, bits=BITS)
        torch.cuda.synchronize()
    print(json.dumps({"prefill_probe": "done"}), flush=True)


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "affine_swiglu_m1_hbm_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the headline kernel from the committed counter summary (the
    line ``traffic_bytes_per_launch: N``), or None when that summary is absent."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


def cpu_baseline(budget_s=12.0):
    """NumPy oracle (variant A: unpack + dequantize + fp32 BLAS every call) on one layer MLP at
    M=1, on this host's cores, for about ``budget_s`` seconds."""
    import numpy as np

    from oracle import affine as O

    try:
        from threadpoolctl import threadpool_info
        threads = max((p.get("num_threads", 1) for p in threadpool_info()), default=1)
    except Exception:  # pragma: no cover - informational only
        threads = os.cpu_count() or 1
    gate = O.make_affine_weight(INTER, HIDDEN, BITS, GROUP, 1, 10)
    up = O.make_affine_weight(INTER, HIDDEN, BITS, GROUP, 1, 12)
    down = O.make_affine_weight(HIDDEN, INTER, BITS, GROUP, 1, 14)
    x = O.make_activations(1, HIDDEN, 1)
    res = O.make_activations(1, HIDDEN, 1, tensor_id=3)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter_ns()
        O.affine_mlp(x, gate, up, down, GROUP, BITS, residual=res, acc=np.float32)
        times.append((time.perf_counter_ns() - t0) / 1e3)
    times.sort()
    us = times[len(times) // 2]
    return {
        "value": round(mlp_bytes(1) / (us * 1e-6) / 1e9, 3),
        "unit": "GB/s",
        "us_per_call": round(us, 1),
        "cores": int(threads),
        "kind": "port",
        "sample": f"NumPy oracle, one INT4 MLP layer (H={HIDDEN}, I={INTER}) at M=1, "
                  f"{len(times)} calls (median), fp32 BLAS, unpack+dequantize every call",
    }


def tuning_report(args):
    """The plan decisions the timed runs took: shape, the planner's plan and the chosen one,
    each timed by the tuner (us per dispatch)."""
    if args.no_tune:
        return {"enabled": False}
    from metile_amd import tuning

    def short(plan):
        if plan is None:
            return "planner"
        return ",".join(f"{k}={v}" for k, v in plan.items())

    decisions = []
    for e in tuning.cached_decisions():
        decisions.append({
            "op": e.get("op"), "rows": e.get("rows"), "K": e.get("input_features"),
            "N": e.get("output_features"), "bits": e.get("bits"), "nproj": e.get("nproj", 1),
            "planner": short(e.get("planner")), "chosen": short(e.get("plan")),
            "planner_us": e.get("planner_us"), "chosen_us": e.get("chosen_us"),
            **({"layout": e["layout"]} if "layout" in e else {})})
    decisions.sort(key=lambda d: (d["op"], d["nproj"], d["K"], d["N"], d["rows"]))
    return {"enabled": True, "switch_margin": tuning.SWITCH_MARGIN, "decisions": decisions}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--headline-only", action="store_true",
                    help="skip the other configs and the read ceiling")
    ap.add_argument("--rows", default=",".join(str(m) for m in ROWS),
                    help="comma-separated row counts of the headline MLP (default: all)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only the eager launches profiled by the HBM-traffic counter runs")
    ap.add_argument("--prefill-probe", action="store_true",
                    help="only eager config-4 GEMM launches, for instruction-counter runs")
    ap.add_argument("--no-tune", action="store_true",
                    help="run every shape on the planner's plan (no plan tuning)")
    args = ap.parse_args()
    if not args.no_tune and "METILE_AMD_CACHE_DIR" not in os.environ:
        # decisions are measured in this run (and reported), not read from an earlier one
        import tempfile

        os.environ["METILE_AMD_CACHE_DIR"] = tempfile.mkdtemp(prefix="metile_amd_bench_")
    if args.gpus != 1:
        print("bench.py measures one GPU only: the hot path runs on a single MI355X and this "
              "build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import metile_amd as mt

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(1234)
    stream = torch.cuda.Stream(device)
    if args.traffic_probe:
        traffic_probe(mt, gen, device, args)
        return
    if args.prefill_probe:
        prefill_probe(mt, gen, device)
        return

    with torch.cuda.stream(stream):
        rows_out, kernel, step_ms = section_mlp(mt, gen, device, stream, args)
        configs, ceiling = {}, None
        if not args.headline_only:
            configs["0"] = section_qmv(mt, gen, device, stream, args, HIDDEN, INTER, 4, ROWS)
            configs["2"] = section_dense(mt, gen, device, stream, args)
            configs["3"] = section_qmv(mt, gen, device, stream, args, 5120, 17408, 8, (1, 8, 16))
            configs["4"] = section_prefill(mt, gen, device, stream, args)
    if not args.headline_only:
        ceiling = section_ceiling(mt, device, stream, args)

    achieved = kernel["swiglu_bytes"] / kernel["swiglu_us"] / 1e3
    value = LAYERS * mlp_bytes(1) / (step_ms * 1e-3) / 1e9
    result = {
        "metric": "INT4 qmv achieved HBM GB/s (% of peak) at M=1..32; us/call for SwiGLU MLP",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 codes, bf16 activations, fp32 accumulate",
        "data": "synthetic seeded weights (BASELINE recipe), 28-layer stack to defeat the MALL",
        "config": {
            "workload": "INT4 fused SwiGLU MLP, Qwen2.5-1.5B shape (H=1536, I=8960, g64), "
                        "M=1 decode row through 28 distinct layers per step (config 1); codes "
                        f"kept in the layout the tuner picked per stage (gate/up "
                        f"{kernel['layouts']['gate_up']}, down {kernel['layouts']['down']}), "
                        "prepared once, ahead of time",
            "layers": LAYERS, "hidden": HIDDEN, "intermediate": INTER, "group_size": GROUP,
            "bits": BITS, "rows": 1,
        },
        "rows": rows_out,
        "roofline": {
            "bound": "hbm",
            "kernel": kernel["swiglu_label"] + " (fused gate/up SwiGLU), M=1",
            "down_kernel": kernel["down_label"],
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "avg_kernel_us": round(kernel["swiglu_us"], 3),
            "bytes_per_launch": kernel["swiglu_bytes"],
            "down_avg_kernel_us": round(kernel["down_us"], 3),
            "down_achieved": round(kernel["down_bytes"] / kernel["down_us"] / 1e3, 1),
        },
        "layouts": kernel["layouts"],
        "native_layout": kernel["native_layout"],
        "tuning": tuning_report(args),
    }
    if configs:
        result["configs"] = configs
    if ceiling:
        result["ceiling"] = {"stream_read_one_launch": ceiling}
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
