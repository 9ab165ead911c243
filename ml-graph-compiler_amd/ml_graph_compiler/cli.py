"""Command line interface: ``python -m ml_graph_compiler <command> MODEL [options]``.

The commands and options follow the reference CLI (src/ml_graph_compiler/cli.py:20-340):
``inspect``, ``optimize``, ``plan`` and ``compile``, a model given as an ONNX file or a bundled
sample/config name, ``--dim NAME=N`` and ``--shape INPUT=D0xD1...`` to bind symbolic input
dimensions. ``compile`` builds with the hip backend (``--backend hip``, the only one in this
build) and runs the model once on the GPU with random inputs. Two reference commands are
absent: ``run`` executes the reference's CPU interpreter and ``mlir`` exports MLIR text; neither
is part of this backend. ``compile --check`` compares against an O0 build of the same model on
the GPU, not against the interpreter.
"""

from __future__ import annotations

import argparse
import json
import sys
from collections.abc import Sequence
from pathlib import Path
from typing import Any

import numpy as np

from . import __version__
from .errors import CompilerError
from .ir import Graph, numpy_dtype


def _parse_dims(items: Sequence[str]) -> dict[str, int]:
    dims: dict[str, int] = {}
    for item in items:
        name, _, value = item.partition("=")
        if not name or not value.isdigit():
            raise CompilerError(f"--dim expects NAME=INT, got {item!r}")
        dims[name] = int(value)
    return dims


def _parse_shapes(items: Sequence[str]) -> dict[str, tuple[int, ...]]:
    shapes: dict[str, tuple[int, ...]] = {}
    for item in items:
        name, _, value = item.partition("=")
        parts = value.lower().split("x") if value else []
        if not name or not parts or not all(p.isdigit() for p in parts):
            raise CompilerError(f"--shape expects NAME=D0xD1x..., got {item!r}")
        shapes[name] = tuple(int(p) for p in parts)
    return shapes


def load_model(args: argparse.Namespace) -> Graph:
    """The model named on the command line: a bundled sample/config name or an ONNX file."""
    from .builders import CONFIGS, SAMPLES
    from .onnx_import import from_onnx

    if args.model in SAMPLES:
        return SAMPLES[args.model]()
    if args.model in CONFIGS:
        return CONFIGS[args.model]()
    if not Path(args.model).exists():
        names = ", ".join(list(SAMPLES) + list(CONFIGS))
        raise CompilerError(f"{args.model!r} is neither a file nor a bundled sample ({names})")
    return from_onnx(Path(args.model), _parse_shapes(args.shape), _parse_dims(args.dim))


_INDEX_PASSTHROUGH = ("Reshape", "Flatten", "Squeeze", "Unsqueeze", "Identity", "Cast")


def _gather_bound(value, depth: int = 0) -> int | None:
    """The smallest extent a Gather indexes with ``value`` (directly or through reshapes and
    casts), so random token ids stay in range; None when nothing gathers with it."""
    bound = None
    for u in value.users:
        if u.op == "Gather" and len(u.inputs) > 1 and u.inputs[1] is value and u.input(0).type is not None:
            data = u.input(0).tensor_type
            axis = int(u.attrs.get("axis", 0))
            size = int(data.shape[axis + data.rank if axis < 0 else axis])
            bound = size if bound is None else min(bound, size)
        elif u.op in _INDEX_PASSTHROUGH and depth < 4:
            inner = _gather_bound(u.output, depth + 1)
            if inner is not None:
                bound = inner if bound is None else min(bound, inner)
    return bound


def random_inputs(graph: Graph, seed: int = 0, int_high: int = 100) -> dict[str, np.ndarray]:
    """Random feeds for every graph input: standard normal floats, integers in [0, int_high)
    (or below the extent a Gather indexes with them, if smaller), random booleans."""
    rng = np.random.default_rng(seed)
    feeds: dict[str, np.ndarray] = {}
    for v in graph.inputs:
        t = v.tensor_type
        dt = numpy_dtype(t.dtype)
        if dt == np.bool_:
            feeds[v.name] = rng.random(t.shape) < 0.5
        elif dt.kind in "iu":
            bound = _gather_bound(v)
            high = int_high if bound is None else max(1, min(int_high, bound))
            feeds[v.name] = rng.integers(0, high, t.shape).astype(dt)
        else:
            feeds[v.name] = rng.standard_normal(t.shape).astype(dt)
    return feeds


def _add_model_args(p: argparse.ArgumentParser) -> None:
    p.add_argument("model", help="ONNX file, bundled sample (mlp, tiny-cnn, tiny-gpt, tiny-bert) or config")
    p.add_argument("--dim", action="append", default=[], metavar="NAME=N",
                   help="value for a symbolic input dimension (repeatable)")
    p.add_argument("--shape", action="append", default=[], metavar="INPUT=D0xD1",
                   help="full static shape for one input (repeatable)")


def _print(payload: dict[str, Any], as_json: bool) -> None:
    if as_json:
        print(json.dumps(payload, indent=2, default=str))
        return
    for key, value in payload.items():
        if isinstance(value, dict):
            print(f"{key}:")
            for k, v in value.items():
                print(f"  {k}: {v}")
        elif isinstance(value, list):
            print(f"{key}:")
            for item in value:
                print(f"  {item}")
        else:
            print(f"{key}: {value}")


def cmd_inspect(args: argparse.Namespace) -> int:
    graph = load_model(args)
    if args.print_ir:
        print(graph)
        return 0
    _print(graph.summary(), args.json)
    return 0


def cmd_optimize(args: argparse.Namespace) -> int:
    from .passes import optimize

    graph = load_model(args)
    before = graph.op_counts()
    report = optimize(graph, args.opt)
    if args.print_ir:
        print(graph)
        return 0
    if args.json:
        _print({"pipeline": args.opt, **report.to_dict(), "ops_before": before, "ops_after": graph.op_counts()}, True)
        return 0
    _print({
        "pipeline": args.opt,
        "nodes": f"{report.nodes_before} -> {report.nodes_after}",
        "passes": [f"{r.name:<9} changes={r.changes:<4} nodes={r.nodes_after:<5} {r.seconds * 1e3:7.1f} ms"
                   for r in report.records],
        "ops before": before,
        "ops after": graph.op_counts(),
    }, False)
    return 0


def cmd_plan(args: argparse.Namespace) -> int:
    from .memory import STRATEGIES, plan_memory
    from .passes import optimize
    from .schedule import schedule

    graph = load_model(args)
    optimize(graph, args.opt)
    report = schedule(graph)
    plans = {s: plan_memory(graph, s, inplace=not args.no_inplace, alignment=args.alignment).summary()
             for s in STRATEGIES}
    if args.json:
        _print({"schedule": report.__dict__, "plans": plans}, True)
        return 0
    mb = 2**20
    _print({
        "nodes": report.nodes,
        "peak live (source order)": f"{report.peak_before / mb:.2f} MB",
        "peak live (scheduled)": f"{report.peak_after / mb:.2f} MB",
        "wavefronts": f"{report.levels} levels, widest {report.max_width}",
        "critical path": f"{report.critical_flops / max(report.total_flops, 1):.1%} of FLOPs",
        "arena by strategy": [
            f"{name:<15} {p['arena_bytes'] / mb:8.2f} MB  (lower bound "  # type: ignore[operator]
            f"{p['lower_bound_bytes'] / mb:.2f} MB, no reuse {p['naive_bytes'] / mb:.2f} MB)"  # type: ignore[operator]
            for name, p in plans.items()
        ],
        "aliases": plans["greedy_by_size"]["aliases"],
        "in place": plans["greedy_by_size"]["inplace"],
    }, False)
    return 0


def _max_diff(got: dict[str, np.ndarray], want: dict[str, np.ndarray]) -> float:
    return max(float(np.max(np.abs(got[k].astype(np.float64) - want[k].astype(np.float64))))
               if want[k].size else 0.0 for k in want)


def cmd_compile(args: argparse.Namespace) -> int:
    from .codegen import compile_graph
    from .passes import optimize
    from .schedule import schedule

    graph = load_model(args)
    feeds = random_inputs(graph, args.seed, args.int_high)
    baseline = None
    if args.check:
        plain = load_model(args)
        optimize(plain, "O0")
        ref_model = compile_graph(plain, cache_dir=args.cache_dir, backend=args.backend, name="model_O0")
        try:
            baseline = ref_model.run(feeds)
        finally:
            ref_model.release()
    optimize(graph, args.opt)
    schedule(graph)
    compiled = compile_graph(graph, cache_dir=args.cache_dir, backend=args.backend)
    report = compiled.report
    assert report is not None
    payload: dict[str, Any] = {
        "backend": report.backend,
        "pipeline": args.opt,
        "library": str(compiled.library_path),
        "source_lines": report.c_lines,
        "kernels": report.kernels,
        "arena_mb": round(report.arena_bytes / 2**20, 2),
        "weights_mb": round(report.weights_bytes / 2**20, 2),
        "codegen_s": report.codegen_seconds,
        "build_s": report.build_seconds,
        "cached": report.cached,
    }
    try:
        outputs = compiled.run(feeds)
        payload["outputs"] = {k: f"{v.dtype}{list(v.shape)} mean={float(v.mean()) if v.size else 0.0:.6f}"
                              for k, v in outputs.items()}
        if baseline is not None:
            payload["max_abs_diff_vs_O0"] = _max_diff(outputs, baseline)
        if args.bench:
            payload["device_ms"] = round(compiled.benchmark_device(feeds, warmup=2, replays=args.bench), 4)
            times = sorted(compiled.benchmark(feeds, warmup=2, repeat=args.bench))
            payload["latency_ms_median"] = round(1000 * times[len(times) // 2], 3)
            payload["latency_ms_min"] = round(1000 * times[0], 3)
        if args.output:
            payload["saved"] = str(compiled.save(args.output))
        if args.emit_source:
            Path(args.emit_source).write_text((compiled.library_path.parent / "model.cpp").read_text())
            payload["host_source"] = args.emit_source
    finally:
        compiled.release()
    _print(payload, args.json)
    return 0


def cmd_export(args: argparse.Namespace) -> int:
    from .onnx_export import save_onnx

    graph = load_model(args)
    path = save_onnx(graph, args.output)
    print(f"wrote {path}: {len(graph.nodes)} nodes, {len(graph.constants())} initializers, opset {graph.opset}")
    return 0


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(prog="mgc", description="Deep learning graph compiler: ONNX in, "
                                     "hip (gfx950) code out.")
    parser.add_argument("--version", action="version", version=f"%(prog)s {__version__}")
    sub = parser.add_subparsers(dest="command", required=True)

    p = sub.add_parser("inspect", help="import a model and summarize the graph")
    _add_model_args(p)
    p.add_argument("--print-ir", action="store_true", help="print the IR text")
    p.add_argument("--json", action="store_true")
    p.set_defaults(fn=cmd_inspect)

    p = sub.add_parser("optimize", help="run a pass pipeline and report the effect of each pass")
    _add_model_args(p)
    p.add_argument("-O", "--opt", default="O3", help="O0..O3, an ablation level, or pass,pass,...")
    p.add_argument("--print-ir", action="store_true", help="print the optimized IR")
    p.add_argument("--json", action="store_true")
    p.set_defaults(fn=cmd_optimize)

    p = sub.add_parser("plan", help="schedule the graph and plan its memory arena")
    _add_model_args(p)
    p.add_argument("-O", "--opt", default="O3")
    p.add_argument("--no-inplace", action="store_true", help="disable in-place reuse")
    p.add_argument("--alignment", type=int, default=256, help="arena offset alignment in bytes")
    p.add_argument("--json", action="store_true")
    p.set_defaults(fn=cmd_plan)

    p = sub.add_parser("compile", help="generate hip host code, build it and run it on the GPU")
    _add_model_args(p)
    p.add_argument("-O", "--opt", default="O3")
    p.add_argument("--backend", default="hip", help="code generator (this build has: hip)")
    p.add_argument("-o", "--output", help="directory to save the library, weights and metadata")
    p.add_argument("--emit-source", metavar="FILE", help="also write the generated host source")
    p.add_argument("--cache-dir", help="build cache (default ~/.cache/ml-graph-compiler-hip)")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--int-high", type=int, default=100, help="upper bound for integer inputs")
    p.add_argument("--check", action="store_true", help="compare against an O0 build of the model")
    p.add_argument("--bench", type=int, default=0, metavar="N", help="time N runs")
    p.add_argument("--json", action="store_true")
    p.set_defaults(fn=cmd_compile)

    p = sub.add_parser("export", help="write a model (e.g. a bundled sample) as an ONNX file")
    _add_model_args(p)
    p.add_argument("-o", "--output", required=True, help="the .onnx file to write")
    p.set_defaults(fn=cmd_export)
    return parser


def main(argv: Sequence[str] | None = None) -> int:
    parser = build_parser()
    args = parser.parse_args(argv)
    try:
        return int(args.fn(args))
    except CompilerError as exc:
        print(f"error: {exc}", file=sys.stderr)
        return 2
