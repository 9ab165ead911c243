#!/usr/bin/env python3
"""Benchmark of the hip backend: ResNet-50 fp32 img/s on one MI355X.

A "step" is one forward pass of the compiled model over one batch of synthetic input (seeded
N(0,1) images, He-normal weights, BatchNorm folded at -O3), replayed as the captured hipGraph
with inputs already resident in HBM. The timed region is exactly ``--steps`` replays between two
stream synchronizations (wall clock, cross-checked with hipEvents on the model stream).

Printed: ONE JSON line with the driver's fields plus
* ``roofline``: the fp32 MFMA GEMM / implicit-GEMM convolution kernels (all conv and FC nodes):
  algorithmic FLOPs per launch (ops.flops of the node, 2 per MAC) over the kernel's average
  duration in graph replays, measured in the run by a rocprofv3 --kernel-trace child over
  ``--trace-probe`` (``duration_source`` says so; ``event_avg_launch_us`` is the eager
  per-node hipEvent figure, and ``--no-trace`` falls back to it); ``traffic`` is the HBM bytes
  per GEMM launch, measured in the run by two rocprofv3 counter runs (FETCH_SIZE, WRITE_SIZE)
  over ``--pmc-probe`` (``traffic_source`` says so, or names the committed summary
  profiles/<workload>_b<batch>_gemm_traffic.md it fell back to);
* ``cpu_baseline``: the reference's generated-C + OpenMP backend (its own C kernels, built from
  the reference sources into oracle/_ref) on this host's cores by the reference's latency
  method (fresh process per cell, 3 interleaved rounds, bootstrap CI) at the GPU batch;
* ``b1``: the same model at batch 1 (latency and img/s).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT), str(ROOT / "ml-graph-compiler_amd")]

import numpy as np  # noqa: E402

MFMA_FP32_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0


def _membench_cases():
    """Single-operator graphs at bandwidth-bound sizes (hundreds of MB per launch) for every
    memory-bound kernel family: (label, graph, feeds, op of the node to time)."""
    from ml_graph_compiler.ir import Graph, TensorType
    from ml_graph_compiler.shape_inference import infer_shapes

    rng = np.random.default_rng(0)

    def f32(*shape):
        return rng.standard_normal(shape, dtype=np.float32)

    cases = []

    def single(label, op, inputs, attrs=None, consts=(), n_out=1, time_op=None):
        g = Graph(label.replace(" ", "_"))
        vals, feeds = [], {}
        for i, arr in enumerate(inputs):
            if i in consts:
                vals.append(g.constant(arr, f"c{i}"))
            else:
                vals.append(g.add_input(f"x{i}", TensorType("float32", arr.shape)))
                feeds[f"x{i}"] = arr
        node = g.add_node(op, vals, n_out, attrs or {}, name="op")
        for j, o in enumerate(node.outputs):
            g.add_output(o, f"y{j}")
        infer_shapes(g)
        cases.append((label, g, feeds, time_op or op))

    rows = 1 << 17
    single("LayerNorm 131072 x 768", "LayerNormalization", [f32(rows, 768), f32(768), f32(768)], {"axis": -1}, consts=(1, 2))
    single("Softmax 65536 x 1024", "Softmax", [f32(1 << 16, 1024)], {"axis": -1})
    single("Add 64M + 64M", "Add", [f32(1 << 26), f32(1 << 26)])
    single("Add 16 x 4096 x 1024 + bias row", "Add", [f32(16, 4096, 1024), f32(1024)])
    single("Gelu 64M", "Gelu", [f32(1 << 26)])
    single("Transpose 8192 x 8192", "Transpose", [f32(8192, 8192)], {"perm": [1, 0]})
    single("Transpose head split 64 x 512 x 12 x 64", "Transpose", [f32(64, 512, 12, 64)], {"perm": [0, 2, 1, 3]})
    single("Depthwise 3x3 s1 32 x 144 x 112 x 112", "Conv",
           [f32(32, 144, 112, 112), f32(144, 1, 3, 3), f32(144)],
           {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 144}, consts=(1, 2), time_op="FusedConv")
    single("Depthwise 3x3 s2 32 x 144 x 112 x 112", "Conv",
           [f32(32, 144, 112, 112), f32(144, 1, 3, 3), f32(144)],
           {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "strides": [2, 2], "group": 144}, consts=(1, 2),
           time_op="FusedConv")
    single("MaxPool 3x3 s2 32 x 128 x 112 x 112", "MaxPool", [f32(32, 128, 112, 112)],
           {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]})
    single("GlobalAveragePool 64 x 2048 x 14 x 14", "GlobalAveragePool", [f32(64, 2048, 14, 14)])
    return cases


def membench(cache: Path, replays: int = 5) -> str:
    """Achieved bandwidth of each memory-bound kernel family at bandwidth-bound sizes: the timed
    node's input + output bytes over its hipEvent duration (eager, best of ``replays``)."""
    from ml_graph_compiler.codegen import compile_graph
    from ml_graph_compiler.ir import numpy_dtype
    from ml_graph_compiler.passes import optimize
    from ml_graph_compiler.schedule import schedule

    def nbytes(v):
        return int(np.prod(v.type.shape)) * np.dtype(numpy_dtype(v.type.dtype)).itemsize

    out = ["| case | timed node | MB moved | us | GB/s | % of 8 TB/s |", "|---|---|---:|---:|---:|---:|"]
    for label, g, feeds, op in _membench_cases():
        log(f"membench {label}")
        optimize(g, "O3")
        schedule(g)
        model = compile_graph(g, cache_dir=cache, name="membench", profile=True)
        try:
            model.upload(feeds)
            model.profile_reset()
            model.profile_run(1)  # warm
            best = None
            for _ in range(replays):
                model.profile_reset()
                model.profile_run(1)
                t = next(sec for (o, _name, sec), node in zip(model.profile(), g.nodes) if o == op)
                best = t if best is None else min(best, t)
        finally:
            model.release()
        node = next(n for n in g.nodes if n.op == op)
        moved = sum(nbytes(v) for v in node.inputs if v is not None) + sum(nbytes(v) for v in node.outputs)
        gbs = moved / best / 1e9
        out.append(f"| {label} | {op} | {moved / 1e6:.1f} | {best * 1e6:.1f} | {gbs:.0f} | {100 * gbs / HBM_PEAK_GBS:.1f} |")
    return "\n".join(out)
WORKLOADS = ("resnet50", "bottleneck", "mobilenet_v2", "bert_base", "gpt2", "single_gemm")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_graph(workload: str, batch: int):
    from ml_graph_compiler import builders

    if workload == "single_gemm":
        return builders.single_gemm()
    return builders.CONFIGS[workload](batch=batch)


def compile_workload(workload: str, batch: int, cache: Path):
    from ml_graph_compiler.codegen import compile_graph
    from ml_graph_compiler.passes import optimize
    from ml_graph_compiler.schedule import schedule

    g = build_graph(workload, batch)
    optimize(g, "O3")
    schedule(g)
    model = compile_graph(g, cache_dir=cache, name=f"{workload}_b{batch}", profile=True)
    return g, model


def feeds_for(graph, seed: int = 0):
    from ml_graph_compiler.builders import random_feeds

    return random_feeds(graph, seed, int_high=30522 if any(v.type.dtype == "int64" for v in graph.inputs) else 100)


def time_replays(model, steps: int) -> tuple[float, float]:
    """(wall seconds, event milliseconds) of ``steps`` graph replays on resident inputs."""
    model.sync()
    t0 = time.perf_counter()
    model.launch(steps)
    model.sync()
    wall = time.perf_counter() - t0
    ev_ms = float(model.lib.mgc_hip_time_graph(int(steps)))
    model.sync()
    return wall, ev_ms


def gemm_roofline(graph, model, replays: int) -> dict:
    """Achieved TFLOP/s of the MFMA GEMM kernels from per-node hipEvent durations."""
    model.profile_reset()
    model.profile_run(replays)
    prof = model.profile()
    flops = 0
    secs = 0.0
    launches = 0
    for (op, _name, sec), node, f in zip(prof, graph.nodes, model.node_flops):
        # f == 0: a GEMM node absorbed into a fused attention call (its work is timed there)
        if op in ("FusedConv", "Conv", "FusedGemm", "Gemm", "MatMul") and not _is_depthwise(node) and f > 0:
            flops += f * replays
            secs += sec
            launches += replays
    total = sum(sec for _, _, sec in prof)
    achieved = flops / secs / 1e12 if secs > 0 else 0.0
    return {
        "bound": "mfma",
        "kernel": ("the fp32 MFMA GEMM family: every GEMM / implicit-GEMM convolution kernel (gemm_dma, "
                   "gemm_dma_tail, gemm_dma_wsplit, gemm_dma_wsplit16, gemm_stream, gemm_mfma, gemm_dw, "
                   "gemm_expand_dw, mbconv), split-K reductions apart"),
        "achieved": round(achieved, 2),
        "peak": MFMA_FP32_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / MFMA_FP32_PEAK_TFLOPS, 4),
        "traffic": None,
        "flops_per_launch": int(flops / max(launches, 1)),
        "avg_launch_us": round(1e6 * secs / max(launches, 1), 2),
        "share_of_forward": round(secs / total, 3) if total > 0 else None,
    }


def _is_depthwise(node) -> bool:
    from ml_graph_compiler.codegen.hip import HipEmitter

    return HipEmitter.depthwise(node)


def cpu_baseline(workload: str, gpu_batch: int) -> dict | None:
    """The reference's generated-C backend on this host's cores, by the reference's latency
    method (oracle/cpu_bench.py: a fresh process per cell, 3 interleaved rounds, bootstrap 95%
    CI of the median): the GPU batch on every core (the reported value), batch 1 on every core
    and on one. Bounded to about a minute of CPU time."""
    try:
        from oracle import cbackend, cpu_bench
    except Exception as exc:  # pragma: no cover - reported, not fatal
        log(f"cpu baseline unavailable: {exc}")
        return None
    if workload == "single_gemm":
        gpu_batch = 1
    batches = cbackend.BASELINES.get(workload, ())
    if gpu_batch not in batches:
        log(f"cpu baseline: no prebuilt reference library for {workload} b{gpu_batch}")
        return None
    info = cpu_bench.host()
    cores = info["nproc"]
    big = gpu_batch > 1
    cells = [(workload, gpu_batch, cores, 1 if big else 5, 3 if big else 30)]
    if big:
        cells.append((workload, 1, cores, 5, 30))
    cells.append((workload, 1, 1, 1, 3))
    try:
        log(f"cpu baseline: {len(cells)} cells x 3 rounds, fresh process each, on {cores} cores of {info['cpu_model']}")
        rows = {(r["batch"], r["threads"]): r for r in cpu_bench.measure(cells, rounds=3)}
    except Exception as exc:
        log(f"cpu baseline failed: {exc}")
        return None
    units = 1 if workload == "single_gemm" else gpu_batch
    unit = {"single_gemm": "calls/s", "bert_base": "seq/s", "gpt2": "seq/s"}.get(workload, "img/s")

    plan = {(b, t): (w, rep) for _, b, t, w, rep in cells}

    def rate(batch: int, threads: int) -> str:
        r = rows[(batch, threads)]
        lo, hi = r["median_ci95_ms"]
        n = 1 if workload == "single_gemm" else batch
        warm, rep = plan[(batch, threads)]
        return (f"b{batch} on {threads} thread(s): {1e3 * n / r['median_ms']:.2f} {unit} (median {r['median_ms']:.1f} ms, "
                f"95% CI {lo:.1f}-{hi:.1f} ms, {r['samples']} runs: warmup {warm} and repeat {rep} per round)")

    head = rows[(gpu_batch, cores)]
    text = "; ".join(rate(b, t) for (b, t) in rows)
    return {
        "value": round(1e3 * units / head["median_ms"], 3),
        "unit": unit,
        "cores": cores,
        "kind": "reference",
        "sample": (f"{workload}: the reference's generated-C + OpenMP backend (its own mgc_kernels.c, -O3 -fopenmp "
                   f"-march=x86-64-v3) on '{info['cpu_model']}' (nproc {cores}); a fresh process per cell, 3 interleaved "
                   f"rounds, bootstrap CI of the median (the reference's benchmarks/latency.py method; its warmup 5 / "
                   f"repeat 30 are cut for the GPU-batch cell and the one-thread cell to keep the run within minutes); "
                   f"{text}"),
        "median_ci95_ms": head["median_ci95_ms"],
    }


def measure_traffic(workload: str, batch: int, cache: Path) -> tuple[int | None, str]:
    """HBM bytes per GEMM launch measured now: two rocprofv3 counter runs (FETCH_SIZE, then
    WRITE_SIZE) over ``--pmc-probe``, each calibrated on the probe's 256 MiB copy. Falls back
    to the committed summary (labelled as recorded) when a run fails."""
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    out = Path(tempfile.mkdtemp(prefix="mgc-pmc-", dir="/tmp"))
    runs = {}
    try:
        if prof is None:
            raise RuntimeError("rocprofv3 not found")
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            d = out / counter.lower()
            cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", str(d), "-o", "p", "--",
                   sys.executable, str(ROOT / "bench.py"), "--pmc-probe", "--workload", workload,
                   "--batch", str(batch), "--cache", str(cache)]
            log(f"traffic: rocprofv3 --pmc {counter} over the probe")
            proc = subprocess.run(cmd, cwd="/tmp", env={**os.environ, "TMPDIR": "/tmp"}, capture_output=True,
                                  text=True, timeout=180, check=False)
            runs[counter] = per_dispatch(d, counter)
            if not runs[counter]:
                raise RuntimeError(f"no {counter} rows (rc {proc.returncode}): {proc.stderr[-400:]}")
        bf, bw, _, _ = calibration(runs["FETCH_SIZE"], runs["WRITE_SIZE"])

        gf = [v for name, v in runs["FETCH_SIZE"] if _is_gemm_kernel(name)]
        gw = [v for name, v in runs["WRITE_SIZE"] if _is_gemm_kernel(name)]
        if not gf or len(gf) != len(gw):
            raise RuntimeError("GEMM dispatch counts differ between the two runs")
        return int(round((bf * sum(gf) + bw * sum(gw)) / len(gf))), (
            "measured in this run: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE over bench.py --pmc-probe, "
            "each scaled by the counter's reading for a 256 MiB copy")
    except Exception as exc:
        log(f"traffic measurement failed ({exc}); using the committed summary")
        return recorded_traffic(workload, batch), f"recorded: {traffic_file(workload, batch).relative_to(ROOT)}"
    finally:
        shutil.rmtree(out, ignore_errors=True)


TRAFFIC_KEY = "traffic_bytes_per_launch:"
CALIBRATION_FLOATS = 1 << 26  # 256 MiB copied by the calibration kernel


def traffic_file(workload: str, batch: int) -> Path:
    return ROOT / "profiles" / f"{workload}_b{batch}_gemm_traffic.md"


def recorded_traffic(workload: str, batch: int) -> int | None:
    """HBM bytes per GEMM launch from the committed counter summary, if there is one."""
    path = traffic_file(workload, batch)
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.strip().startswith(TRAFFIC_KEY):
            return int(line.split(":", 1)[1].strip())
    return None


def pmc_probe(workload: str, batch: int, cache: Path) -> None:
    """The program the counter runs profile: one plain copy of CALIBRATION_FLOATS floats (a
    single-node O0 graph whose Transpose lowers to the 16-byte copy kernel), then one eager
    forward of the workload with every node launched on its own."""
    from ml_graph_compiler.codegen import compile_graph
    from ml_graph_compiler.ir import Graph, TensorType
    from ml_graph_compiler.shape_inference import infer_shapes

    g = Graph("calibration")
    x = g.add_input("x", TensorType("float32", (CALIBRATION_FLOATS,)))
    node = g.add_node("Transpose", [x], attrs={"perm": [0]})
    g.add_output(node.output, "y")
    infer_shapes(g)
    cal = compile_graph(g, cache_dir=cache, name="calibration_copy", profile=True)
    cal.upload({"x": np.zeros(CALIBRATION_FLOATS, np.float32)})
    cal.profile_run(1)
    cal.sync()
    cal.release()
    graph, model = compile_workload(workload, batch, cache)
    model.upload(feeds_for(graph))
    model.profile_run(1)
    model.sync()
    model.release()
    log("pmc probe done: calibration copy, then one eager forward")


TRACE_REPLAYS = 20


def trace_probe(workload: str, batch: int, cache: Path) -> None:
    """The program the kernel-trace run profiles: TRACE_REPLAYS graph replays of the workload on
    resident inputs after a warmup, the conditions of the timed region."""
    graph, model = compile_workload(workload, batch, cache)
    model.upload(feeds_for(graph))
    model.launch(3)
    model.sync()
    model.launch(TRACE_REPLAYS)
    model.sync()
    model.release()
    log(f"trace probe done: {TRACE_REPLAYS} graph replays")


def _is_gemm_kernel(name: str) -> bool:
    """The GEMM family: every GEMM / implicit-GEMM kernel (the whole-block mbconv kernel is the
    projection GEMM with its producers fused), not the split-K reductions."""
    return ("gemm_" in name or "mbconv_kernel" in name) and "splitk" not in name


def traced_gemm_launch(workload: str, batch: int, cache: Path) -> dict | None:
    """Average duration of the GEMM-family kernels (and per GEMM node with its split-K
    reduction) over TRACE_REPLAYS graph replays, from a rocprofv3 --kernel-trace child run of
    --trace-probe: the duration roofline.achieved divides by."""
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if prof is None:
        log("kernel trace: rocprofv3 not found")
        return None
    out = Path(tempfile.mkdtemp(prefix="mgc-trace-", dir="/tmp"))
    try:
        cmd = [prof, "--kernel-trace", "--output-format", "csv", "-d", str(out), "-o", "p", "--",
               sys.executable, str(ROOT / "bench.py"), "--trace-probe", "--workload", workload,
               "--batch", str(batch), "--cache", str(cache)]
        log("kernel trace: rocprofv3 --kernel-trace over the graph-replay probe")
        proc = subprocess.run(cmd, cwd="/tmp", env={**os.environ, "TMPDIR": "/tmp"}, capture_output=True,
                              text=True, timeout=300, check=False)
        rows = []
        for f in sorted(out.rglob("*kernel_trace.csv")):
            for r in csv.DictReader(open(f)):
                rows.append((r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3))
        gemm = [us for name, us in rows if _is_gemm_kernel(name)]
        red = [us for name, us in rows if "splitk" in name]
        if not gemm:
            raise RuntimeError(f"no GEMM dispatches traced (rc {proc.returncode}): {proc.stderr[-300:]}")
        return {"launches": len(gemm), "avg_us": sum(gemm) / len(gemm),
                "avg_us_with_reductions": (sum(gemm) + sum(red)) / len(gemm), "reductions": len(red)}
    except Exception as exc:
        log(f"kernel trace failed: {exc}")
        return None
    finally:
        shutil.rmtree(out, ignore_errors=True)


def per_dispatch(d: Path, counter: str) -> list[tuple[str, float]]:
    """(kernel name, counter value) of every dispatch of a rocprofv3 --pmc run, in dispatch order."""
    import csv

    rows = []
    for f in sorted(d.rglob("*counter_collection.csv")):
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] == counter:
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return [(name, v) for _, name, v in rows]


def calibration(fetch: list[tuple[str, float]], write: list[tuple[str, float]]) -> tuple[float, float, float, float]:
    """Bytes per counter KiB for FETCH_SIZE and WRITE_SIZE, from the probe's calibration copy
    (the first copy_kernel dispatch), and the raw counter values of that copy."""
    nbytes = 4 * CALIBRATION_FLOATS
    cal_f = next(v for name, v in fetch if "copy_kernel" in name)
    cal_w = next(v for name, v in write if "copy_kernel" in name)
    return nbytes / cal_f, nbytes / cal_w, cal_f, cal_w


def pmc_summary(fetch_dir: Path, write_dir: Path, workload: str, batch: int) -> str:
    """Markdown summary of the FETCH_SIZE and WRITE_SIZE runs over --pmc-probe."""
    fetch = per_dispatch(fetch_dir, "FETCH_SIZE")
    write = per_dispatch(write_dir, "WRITE_SIZE")
    nbytes = 4 * CALIBRATION_FLOATS
    bf, bw, cal_f, cal_w = calibration(fetch, write)
    kf, kw = bf / 1024.0, bw / 1024.0

    gf = [v for name, v in fetch if _is_gemm_kernel(name)]
    gw = [v for name, v in write if _is_gemm_kernel(name)]
    n = len(gf)
    fetch_b = kf * 1024.0 * sum(gf) / n
    write_b = kw * 1024.0 * sum(gw) / n
    per_launch = int(round(fetch_b + write_b))
    # algorithmic bytes: every operand (activations, weights, bias, residual) and the output once
    from ml_graph_compiler.ir import numpy_dtype
    from ml_graph_compiler.passes import optimize

    from ml_graph_compiler.codegen.hip import FUSE_PROJECTION_SHORTCUT, find_projection_shortcuts
    from ml_graph_compiler.schedule import schedule

    g = build_graph(workload, batch)
    optimize(g, "O3")
    schedule(g)

    def nbytes_of(v) -> int:
        return int(np.prod(v.type.shape)) * np.dtype(numpy_dtype(v.type.dtype)).itemsize

    algo = 0
    for node in g.nodes:
        if node.op in ("FusedConv", "Conv", "FusedGemm", "Gemm", "MatMul") and not _is_depthwise(node):
            algo += sum(nbytes_of(v) for v in [v for v in node.inputs if v is not None] + list(node.outputs))
    # a projection shortcut computed inside its block's last GEMM never writes (nor has read back)
    # its output
    shortcuts = find_projection_shortcuts(g) if FUSE_PROJECTION_SHORTCUT else {}
    algo -= sum(2 * nbytes_of(ds.output) for ds in shortcuts.values())
    algo_b = algo / max(n, 1)
    return "\n".join([
        f"# HBM traffic of the GEMM kernels: {workload} b{batch} forward (hip backend, -O3)",
        "",
        "Commands (repo root, on the MI355X box; one counter per run):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp",
        f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d $GRAFT_REPO_ROOT/gpurun_out/pmc_fetch -o p -- python3 $GRAFT_REPO_ROOT/bench.py --pmc-probe --workload {workload} --batch {batch}",
        f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d $GRAFT_REPO_ROOT/gpurun_out/pmc_write -o p -- python3 $GRAFT_REPO_ROOT/bench.py --pmc-probe --workload {workload} --batch {batch}",
        f"python3 bench.py --pmc-summary gpurun_out/pmc_fetch gpurun_out/pmc_write --workload {workload} --batch {batch}",
        "```",
        "",
        f"Calibration: a plain 16-byte copy of {nbytes} bytes read {cal_f:.0f} KiB (FETCH_SIZE) and wrote "
        f"{cal_w:.0f} KiB (WRITE_SIZE); scale factors {kf:.4f} (fetch) and {kw:.4f} (write) turn each "
        "counter into bytes.",
        "",
        f"GEMM dispatches in one eager forward: {n}. Average per launch: fetched {fetch_b / 1e6:.2f} MB, "
        f"written {write_b / 1e6:.2f} MB; the algorithmic minimum (each operand and the output moved "
        f"once; a projection shortcut computed in its block's last GEMM has no output of its own) is "
        f"{algo_b / 1e6:.2f} MB per launch, so HBM traffic is {(fetch_b + write_b) / algo_b:.2f}x it.",
        "",
        f"{TRAFFIC_KEY} {per_launch}",
        "",
    ])


HBM_PEAK_GBS = 8000.0


def _short_kernel(name: str) -> str:
    """Kernel name without its parameter list and namespace (template arguments kept)."""
    name = name.replace("(anonymous namespace)::", "")
    return name.split("(", 1)[0].replace("void ", "").replace("mgc::", "").strip()


def hbm_summary(fetch_dir: Path, write_dir: Path, trace_dir: Path, workload: str, batch: int) -> str:
    """Achieved HBM bandwidth of every kernel of one eager forward: the calibrated FETCH_SIZE +
    WRITE_SIZE bytes of each dispatch (two --pmc runs over --pmc-probe) over the dispatch's
    duration in a third, kernel-trace-only run of the same program. The three runs launch the
    same kernels in the same order; dispatches are matched by position and checked by name."""
    import csv

    fetch = per_dispatch(fetch_dir, "FETCH_SIZE")
    write = per_dispatch(write_dir, "WRITE_SIZE")
    trace = []
    for f in sorted(trace_dir.rglob("*kernel_trace.csv")):
        for r in csv.DictReader(open(f)):
            trace.append((int(r["Dispatch_Id"]), r["Kernel_Name"],
                          (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9))
    trace.sort()
    bf, bw, _, _ = calibration(fetch, write)

    def from_calibration(rows):
        i = next(k for k, r in enumerate(rows) if "copy_kernel" in r[1 if len(r) == 3 else 0])
        return rows[i + 1:]

    def kernels_only(rows):  # the runtime's own blit kernels (uploads) are not the model's
        return [r for r in rows if not r[1 if len(r) == 3 else 0].startswith("__amd_rocclr")]

    fetch, write = kernels_only(from_calibration(fetch)), kernels_only(from_calibration(write))
    trace = kernels_only(from_calibration(trace))
    n = min(len(fetch), len(write), len(trace))
    mismatched = sum(1 for i in range(n) if not (fetch[i][0] == write[i][0] == trace[i][1]))
    if mismatched or not (len(fetch) == len(write) == len(trace)):
        raise SystemExit(f"runs differ: {len(fetch)}/{len(write)}/{len(trace)} dispatches, {mismatched} names differ")
    rows = []
    for i in range(n):
        name = _short_kernel(trace[i][1])
        fb, wb, sec = fetch[i][1] * bf, write[i][1] * bw, trace[i][2]
        rows.append((name, fb, wb, sec))

    def bound(name: str) -> str:
        # the split-K reductions move bytes; the streaming short-K GEMM and the depthwise GEMM
        # (a 3 x 3 depthwise pass feeding a narrow projection) are HBM-bound by design. A whole
        # inverted-residual block (mbconv_kernel) does 53-57 algorithmic FLOP per byte it moves
        # (expansion, depthwise and projection per output pixel against its input, output and
        # residual), above the 19.7 FLOP/B ridge: MFMA-bound.
        if "mbconv" in name:
            return "MFMA"
        if "gemm_" in name and "splitk" not in name and "gemm_stream" not in name and "gemm_dw" not in name:
            return "MFMA"
        return "MFMA/latency" if "attention" in name else "HBM"

    fam: dict[str, list] = {}
    for name, fb, wb, sec in rows:
        a = fam.setdefault(name, [0, 0.0, 0.0])
        a[0] += 1
        a[1] += fb + wb
        a[2] += sec
    total_sec = sum(r[3] for r in rows)
    cmd_base = "$GRAFT_REPO_ROOT/bench.py --pmc-probe --workload {w} --batch {b}".format(w=workload, b=batch)
    out = [
        f"# Achieved HBM bandwidth per kernel: {workload} b{batch} forward (hip backend, -O3)",
        "",
        "Commands (repo root, on the MI355X box; one counter per run, then a kernel trace):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp",
        f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d $GRAFT_REPO_ROOT/gpurun_out/hbm_fetch -o p -- python3 {cmd_base}",
        f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d $GRAFT_REPO_ROOT/gpurun_out/hbm_write -o p -- python3 {cmd_base}",
        f"rocprofv3 --kernel-trace --output-format csv -d $GRAFT_REPO_ROOT/gpurun_out/hbm_trace -o p -- python3 {cmd_base}",
        f"python3 bench.py --hbm-summary gpurun_out/hbm_fetch gpurun_out/hbm_write gpurun_out/hbm_trace --workload {workload} --batch {batch}",
        "```",
        "",
        f"Bytes are FETCH_SIZE and WRITE_SIZE (KiB) scaled by a plain 256 MiB copy in the same program "
        f"(x{bf / 1024:.4f} and x{bw / 1024:.4f}); durations are the kernel trace's "
        f"end - start of the same dispatch. {n} dispatches, {total_sec * 1e6:.1f} us of kernel time. "
        f"GB/s = (fetched + written bytes) / duration; peak {HBM_PEAK_GBS:.0f} GB/s.",
        "",
        "| kernel | bound | launches | MB per launch | avg us | GB/s | % of HBM peak | % of time |",
        "|---|---|---:|---:|---:|---:|---:|---:|",
    ]
    for name, (cnt, nbytes, sec) in sorted(fam.items(), key=lambda kv: -kv[1][2]):
        gbs = nbytes / sec / 1e9
        out.append(f"| `{name}` | {bound(name)} | {cnt} | {nbytes / cnt / 1e6:.2f} | {sec / cnt * 1e6:.2f} | "
                   f"{gbs:.0f} | {100 * gbs / HBM_PEAK_GBS:.1f} | {100 * sec / total_sec:.1f} |")
    out += ["", "Memory-bound dispatches of more than 4 MB, in launch order:", "",
            "| # | kernel | MB fetched | MB written | us | GB/s | % of peak |", "|---:|---|---:|---:|---:|---:|---:|"]
    for i, (name, fb, wb, sec) in enumerate(rows):
        if bound(name) == "HBM" and fb + wb > 4e6:
            gbs = (fb + wb) / sec / 1e9
            out.append(f"| {i} | `{name}` | {fb / 1e6:.2f} | {wb / 1e6:.2f} | {sec * 1e6:.2f} | {gbs:.0f} | "
                       f"{100 * gbs / HBM_PEAK_GBS:.1f} |")
    hb = [(fb + wb, sec) for name, fb, wb, sec in rows if bound(name) == "HBM"]
    if hb:
        nb, ns = sum(b for b, _ in hb), sum(t for _, t in hb)
        out += ["", f"All memory-bound dispatches together: {nb / 1e6:.1f} MB in {ns * 1e6:.1f} us = "
                    f"{nb / ns / 1e9:.0f} GB/s ({100 * nb / ns / 1e9 / HBM_PEAK_GBS:.1f}% of peak).", ""]
    return "\n".join(out)


MI355X_CLOCK_HZ = 2.4e9
MI355X_SIMDS = 256 * 4
MFMA_COUNTERS = "SQ_INSTS_VALU_MFMA_MOPS_F32 SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE"


def kernel_summary(trace_dir: Path, workload: str, batch: int) -> str:
    """Per-kernel durations of graph replays: a rocprofv3 --kernel-trace run of --trace-probe
    (3 warmup + TRACE_REPLAYS replays, nothing else on the GPU apart from the upload copies),
    averaged per forward, with the GEMM family's algorithmic TFLOP/s (node FLOPs from the
    compiled graph, a fused projection shortcut or depthwise convolution counted at the launch
    that computes it)."""
    import csv

    from ml_graph_compiler.codegen import build as native
    from ml_graph_compiler.codegen.hip import generate_hip

    rows = []
    for f in sorted(trace_dir.rglob("*kernel_trace.csv")):
        for r in csv.DictReader(open(f)):
            if r["Kernel_Name"].startswith("__amd_rocclr"):
                continue
            rows.append((int(r["Dispatch_Id"]), _short_kernel(r["Kernel_Name"]),
                         (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9))
    rows.sort()
    forwards = 3 + TRACE_REPLAYS
    fam: dict[str, list] = {}
    for _, name, sec in rows:
        a = fam.setdefault(name, [0, 0.0])
        a[0] += 1
        a[1] += sec
    total = sum(sec for _, _, sec in rows) / forwards
    g = build_graph(workload, batch)
    from ml_graph_compiler.passes import optimize
    from ml_graph_compiler.schedule import schedule

    optimize(g, "O3")
    schedule(g)
    gen = generate_hip(g, gemm_workspace=native.gemm_workspace_floats,
                       gemm_ln_workspace=native.gemm_layer_norm_workspace_floats)
    gemm_flops = gen.gemm_flops
    gemm_sec = sum(sec for _, name, sec in rows if _is_gemm_kernel(name)) / forwards
    gemm_n = sum(1 for _, name, _ in rows if _is_gemm_kernel(name)) / forwards
    label = "128 rows" if workload == "single_gemm" else f"batch {batch}"
    out = [
        f"# Kernels of one forward in graph replays: {workload} ({label}, hip backend, -O3)",
        "",
        "Commands (repo root, on the MI355X box):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp",
        f"rocprofv3 --kernel-trace --stats --output-format csv -d $GRAFT_REPO_ROOT/gpurun_out/kt_{workload}_b{batch} -o p -- "
        f"python3 $GRAFT_REPO_ROOT/bench.py --trace-probe --workload {workload} --batch {batch}",
        f"python3 bench.py --kernel-summary gpurun_out/kt_{workload}_b{batch} --workload {workload} --batch {batch}",
        "```",
        "",
        f"The probe replays the captured forward {forwards} times (3 warmup + {TRACE_REPLAYS}) on resident inputs; "
        f"durations are the kernel trace's end - start of each dispatch, averaged per forward. Kernel time per "
        f"forward: {total * 1e6:.1f} us in {len(rows) / forwards:.0f} launches.",
        "",
        "| kernel | launches per forward | avg us | us per forward | % of forward |",
        "|---|---:|---:|---:|---:|",
    ]
    for name, (cnt, sec) in sorted(fam.items(), key=lambda kv: -kv[1][1]):
        out.append(f"| `{name}` | {cnt / forwards:g} | {sec / cnt * 1e6:.2f} | {sec / forwards * 1e6:.1f} | "
                   f"{100 * sec / forwards / total:.1f} |")
    if gemm_n:
        tf = gemm_flops / gemm_sec / 1e12
        out += ["", f"GEMM family (every GEMM / implicit-GEMM kernel, split-K reductions apart): {gemm_n:g} launches "
                    f"per forward, {gemm_sec / gemm_n * 1e6:.2f} us average, {gemm_flops / 1e9:.2f} GFLOP algorithmic "
                    f"per forward -> {tf:.1f} TFLOP/s = {100 * tf / MFMA_FP32_PEAK_TFLOPS:.1f}% of the "
                    f"{MFMA_FP32_PEAK_TFLOPS} TFLOP/s fp32 MFMA peak."]
        stats = []
        for f in sorted(trace_dir.rglob("*kernel_stats.csv")):
            stats += [(r["Name"], int(r["Calls"]), float(r["TotalDurationNs"])) for r in csv.DictReader(open(f))]
        calls = sum(c for name, c, _ in stats if _is_gemm_kernel(name))
        if calls:
            ns = sum(t for name, _, t in stats if _is_gemm_kernel(name))
            out += ["", f"rocprofv3 --stats of the same run (kernel_stats.csv): GEMM family {calls} calls, "
                        f"{ns / calls / 1e3:.2f} us average (all {forwards} forwards)."]
        out.append("")
    return "\n".join(out)


def mfma_summary(pmc_dir: Path, trace_dir: Path, workload: str, batch: int) -> str:
    """MFMA work and utilisation of every matrix-core dispatch of one eager forward: one counter
    run over --pmc-probe (MFMA_COUNTERS) and the kernel-trace run of the same program for
    durations, matched by position and checked by name. SQ_INSTS_VALU_MFMA_MOPS_F32 counts fp32
    MFMA work in units of 512 FLOP; SQ_VALU_MFMA_BUSY_CYCLES counts matrix-core busy cycles,
    reported here per CU per GPU-active cycle (GRBM_GUI_ACTIVE)."""
    import csv

    counters: dict[int, dict] = {}
    for f in sorted(pmc_dir.rglob("*counter_collection.csv")):
        for r in csv.DictReader(open(f)):
            d = counters.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"]})
            d[r["Counter_Name"]] = float(r["Counter_Value"])
    trace = []
    for f in sorted(trace_dir.rglob("*kernel_trace.csv")):
        for r in csv.DictReader(open(f)):
            trace.append((int(r["Dispatch_Id"]), r["Kernel_Name"],
                          (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9))
    trace.sort()
    rows = [counters[k] for k in sorted(counters)]

    def model_only(seq, name_of):
        i = next(k for k, r in enumerate(seq) if "copy_kernel" in name_of(r))
        return [r for r in seq[i + 1:] if not name_of(r).startswith("__amd_rocclr")]

    rows = model_only(rows, lambda r: r["name"])
    trace = model_only(trace, lambda r: r[1])
    if len(rows) != len(trace) or any(a["name"] != b[1] for a, b in zip(rows, trace)):
        raise SystemExit(f"runs differ: {len(rows)} counter dispatches vs {len(trace)} traced")
    fam: dict[str, list] = {}
    tot_flop = tot_sec = 0.0
    for r, (_, name, sec) in zip(rows, trace):
        flop = 512.0 * r.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0)
        if flop <= 0:
            continue
        busy = r.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (sec * MI355X_CLOCK_HZ * MI355X_SIMDS)
        a = fam.setdefault(_short_kernel(name), [0, 0.0, 0.0, 0.0])
        a[0] += 1
        a[1] += flop
        a[2] += sec
        a[3] += busy * sec
        tot_flop += flop
        tot_sec += sec
    base = f"$GRAFT_REPO_ROOT/bench.py --pmc-probe --workload {workload} --batch {batch}"
    out = [
        f"# MFMA work and utilisation: {workload} b{batch} forward (hip backend, -O3)",
        "",
        "Commands (repo root, on the MI355X box; one counter run, then a kernel trace):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp",
        f"rocprofv3 --pmc {MFMA_COUNTERS} --output-format csv -d $GRAFT_REPO_ROOT/gpurun_out/mfma_pmc -o p -- python3 {base}",
        f"rocprofv3 --kernel-trace --output-format csv -d $GRAFT_REPO_ROOT/gpurun_out/hbm_trace -o p -- python3 {base}",
        f"python3 bench.py --mfma-summary gpurun_out/mfma_pmc gpurun_out/hbm_trace --workload {workload} --batch {batch}",
        "```",
        "",
        "FLOP = 512 x SQ_INSTS_VALU_MFMA_MOPS_F32 (the fp32 MFMA work the matrix cores executed, "
        "padding of partial tiles included); TFLOP/s = that over the traced duration; % of peak "
        f"against {MFMA_FP32_PEAK_TFLOPS} TFLOP/s. MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES over the "
        "traced duration x 2.4 GHz x 1024 SIMDs (256 CUs x 4), time-weighted: the fraction of "
        "matrix-core cycles in use. (GRBM_GUI_ACTIVE, summed over the 8 XCDs and stretched by the "
        "counter collection, is not used as the time base.)",
        "",
        "| kernel | launches | GFLOP per launch | avg us | TFLOP/s | % of peak | MFMA busy per SIMD |",
        "|---|---:|---:|---:|---:|---:|---:|",
    ]
    for name, (cnt, flop, sec, busy_sec) in sorted(fam.items(), key=lambda kv: -kv[1][2]):
        tf = flop / sec / 1e12
        out.append(f"| `{name}` | {cnt} | {flop / cnt / 1e9:.3f} | {sec / cnt * 1e6:.2f} | {tf:.1f} | "
                   f"{100 * tf / MFMA_FP32_PEAK_TFLOPS:.1f} | {busy_sec / sec:.3f} |")
    if tot_sec > 0:
        tf = tot_flop / tot_sec / 1e12
        out += ["", f"All MFMA dispatches: {tot_flop / 1e9:.1f} GFLOP in {tot_sec * 1e6:.1f} us = {tf:.1f} TFLOP/s "
                    f"({100 * tf / MFMA_FP32_PEAK_TFLOPS:.1f}% of peak)."]
        from ml_graph_compiler import ops
        from ml_graph_compiler.passes import optimize

        g = build_graph(workload, batch)
        optimize(g, "O3")
        algo = sum(ops.flops(n) for n in g.nodes
                   if n.op in ("FusedConv", "Conv", "FusedGemm", "Gemm", "MatMul") and not _is_depthwise(n))
        out += [f"Algorithmic FLOPs of the graph's contractions (2 per multiply-add): {algo / 1e9:.1f} GFLOP; "
                f"the matrix cores executed {tot_flop / algo:.3f}x that (partial-tile padding, the stem's "
                "space-to-depth zero taps).", ""]
    return "\n".join(out)


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", choices=WORKLOADS, default="resnet50")
    p.add_argument("--batch", type=int, default=32)
    p.add_argument("--profile-replays", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-traffic", action="store_true", help="report the committed traffic summary instead of measuring")
    p.add_argument("--no-b1", action="store_true")
    p.add_argument("--cache", default=os.environ.get("MGC_BENCH_CACHE", "/tmp/mgc-bench-cache"))
    p.add_argument("--pmc-probe", action="store_true", help="run the counter-run program and exit")
    p.add_argument("--trace-probe", action="store_true", help="run the kernel-trace program (graph replays) and exit")
    p.add_argument("--no-trace", action="store_true",
                   help="time the GEMM launches with eager hipEvents instead of a rocprofv3 kernel trace")
    p.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                   help="summarize the FETCH_SIZE / WRITE_SIZE runs into profiles/ and exit")
    p.add_argument("--hbm-summary", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "TRACE_DIR"),
                   help="per-kernel achieved HBM GB/s from two counter runs and a kernel trace of "
                        "--pmc-probe, written to profiles/ and printed")
    p.add_argument("--mfma-summary", nargs=2, metavar=("PMC_DIR", "TRACE_DIR"),
                   help="per-kernel MFMA FLOP, TFLOP/s and busy cycles from a counter run and a "
                        "kernel trace of --pmc-probe, written to profiles/ and printed")
    p.add_argument("--kernel-summary", metavar="TRACE_DIR",
                   help="per-kernel durations of graph replays from a kernel trace of --trace-probe, written "
                        "to profiles/ and printed")
    p.add_argument("--membench", action="store_true",
                   help="achieved HBM bandwidth of every memory-bound kernel family at large sizes; prints a table")
    args = p.parse_args()
    if args.membench:
        print(membench(Path(args.cache)))
        return 0
    if args.kernel_summary:
        batch = 128 if args.workload == "single_gemm" else args.batch
        text = kernel_summary(Path(args.kernel_summary), args.workload, batch)
        (ROOT / "profiles" / f"{args.workload}_b{batch}_kernels.md").write_text(text)
        print(text)
        return 0
    if args.mfma_summary:
        batch = 128 if args.workload == "single_gemm" else args.batch
        text = mfma_summary(*map(Path, args.mfma_summary), args.workload, batch)
        (ROOT / "profiles" / f"{args.workload}_b{batch}_mfma_utilisation.md").write_text(text)
        print(text)
        return 0
    if args.hbm_summary:
        batch = 128 if args.workload == "single_gemm" else args.batch
        text = hbm_summary(*map(Path, args.hbm_summary), args.workload, batch)
        (ROOT / "profiles" / f"{args.workload}_b{batch}_hbm_bandwidth.md").write_text(text)
        print(text)
        return 0
    if args.pmc_summary:
        text = pmc_summary(Path(args.pmc_summary[0]), Path(args.pmc_summary[1]), args.workload, args.batch)
        traffic_file(args.workload, args.batch).write_text(text)
        print(text)
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: every GPU box here has one MI355X; "
                                   "use --gpus 1. Across GPUs the path shards by batch: each GPU replays the same captured "
                                   "graph on its share of the images or sequences with the weights replicated, and no "
                                   "device collective is needed"}))
        return 2
    cache = Path(args.cache)
    batch = 128 if args.workload == "single_gemm" else args.batch
    if args.pmc_probe:
        pmc_probe(args.workload, batch, cache)
        return 0
    if args.trace_probe:
        trace_probe(args.workload, batch, cache)
        return 0

    log(f"compiling {args.workload} b{batch} (O3, hip)")
    graph, model = compile_workload(args.workload, batch, cache)
    feeds = feeds_for(graph)
    model.upload(feeds)
    log(f"warmup {args.warmup}")
    model.launch(args.warmup)
    model.sync()
    log(f"timing {args.steps} replays")
    wall, ev_ms = time_replays(model, args.steps)
    ms_per_step = 1e3 * wall / args.steps
    units = 1 if args.workload == "single_gemm" else batch
    value = units * args.steps / wall
    log(f"{ms_per_step:.3f} ms/step (events {ev_ms / args.steps:.3f} ms), {value:.1f} units/s")
    roof = gemm_roofline(graph, model, args.profile_replays)
    total_flops = sum(model.node_flops)
    model.release()
    traced = None if args.no_trace else traced_gemm_launch(args.workload, batch, cache)
    if traced is not None:
        # the kernel's own duration in graph replays, from the kernel trace; the eager per-node
        # hipEvent figure (event overhead included) is kept beside it
        flops = roof["flops_per_launch"]
        roof["event_avg_launch_us"] = roof["avg_launch_us"]
        roof["avg_launch_us"] = round(traced["avg_us"], 2)
        roof["achieved"] = round(flops / traced["avg_us"] / 1e6, 2)
        roof["frac"] = round(roof["achieved"] / MFMA_FP32_PEAK_TFLOPS, 4)
        roof["achieved_with_reductions"] = round(flops / traced["avg_us_with_reductions"] / 1e6, 2)
        roof["duration_source"] = (f"rocprofv3 --kernel-trace over {TRACE_REPLAYS} graph replays "
                                   f"({traced['launches']} GEMM dispatches, {traced['reductions']} split-K reductions)")
    else:
        roof["duration_source"] = "eager per-node hipEvent pairs on the model stream"
    if args.no_traffic:
        roof["traffic"], roof["traffic_source"] = recorded_traffic(args.workload, batch), "recorded (--no-traffic)"
    else:
        roof["traffic"], roof["traffic_source"] = measure_traffic(args.workload, batch, cache)
    log(f"roofline {roof}")

    b1 = None
    if args.workload in ("resnet50", "bottleneck", "mobilenet_v2", "bert_base", "gpt2") and not args.no_b1 and batch != 1:
        g1, m1 = compile_workload(args.workload, 1, cache)
        m1.upload(feeds_for(g1))
        m1.launch(args.warmup)
        m1.sync()
        w1, e1 = time_replays(m1, max(args.steps, 50))
        n1 = max(args.steps, 50)
        b1 = {"ms_per_step": round(1e3 * w1 / n1, 4), "event_ms_per_step": round(e1 / n1, 4),
              "value": round(n1 / w1, 2)}
        m1.release()
        log(f"b1 {b1}")

    cpu = None if args.no_cpu_baseline else cpu_baseline(args.workload, units)
    unit = {"resnet50": "img/s", "bottleneck": "img/s", "mobilenet_v2": "img/s", "bert_base": "seq/s",
            "gpt2": "seq/s", "single_gemm": "calls/s"}[args.workload]
    line = {
        "metric": "ResNet-50 fp32 img/s at b1/b32; achieved TFLOP/s vs fp32 MFMA peak"
        if args.workload == "resnet50" else f"{args.workload} fp32 {unit}",
        "value": round(value, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "event_ms_per_step": round(ev_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) inputs, random He-normal weights, BN folded at -O3)",
        "config": {"workload": args.workload, "batch": units if args.workload != "single_gemm" else 1,
                   "opt": "O3", "backend": "hip", "achieved_tflops_forward": round(total_flops * value / units / 1e12, 2)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "b1": b1,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
