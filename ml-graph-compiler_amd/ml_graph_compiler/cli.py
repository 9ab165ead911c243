"""``python -m ml_graph_compiler compile MODEL --backend hip``: compile a model for the GPU.

The reference's ``mgc compile`` (src/ml_graph_compiler/cli.py:194-250) with its backend switch:
the model is an ONNX file or a bundled sample/config name, ``--dim NAME=N`` / ``--shape
INPUT=D0xD1...`` bind symbolic input dimensions, ``-O`` picks the pass pipeline. The command
builds the hip model, runs it once on random inputs (integer inputs that index a Gather stay
below its table size) and prints a report; ``--check`` adds the largest difference from the
unoptimized graph evaluated node by node on the CPU, ``--bench N`` times N runs, ``-o DIR``
saves the compiled model. The reference's other commands (inspect, optimize, plan, run, mlir)
are not part of this backend.
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
from .ir import Graph, Value, numpy_dtype


def _bindings(items: Sequence[str], flag: str, shape: bool) -> dict[str, Any]:
    out: dict[str, Any] = {}
    for item in items:
        name, _, text = item.partition("=")
        parts = text.lower().split("x") if shape and text else [text]
        if not name or not all(p.isdigit() for p in parts):
            expected = "NAME=D0xD1x..." if shape else "NAME=INT"
            raise CompilerError(f"{flag} expects {expected}, got {item!r}")
        out[name] = tuple(int(p) for p in parts) if shape else int(parts[0])
    return out


def load_model(model: str, shapes: Sequence[str] = (), dims: Sequence[str] = ()) -> Graph:
    """A bundled sample/config by name, or an ONNX file with its symbolic dimensions bound."""
    from .builders import CONFIGS, SAMPLES
    from .onnx_import import from_onnx

    named = {**SAMPLES, **CONFIGS}
    if model in named:
        return named[model]()
    if not Path(model).exists():
        raise CompilerError(f"{model!r} is neither a file nor a bundled sample ({', '.join(named)})")
    return from_onnx(model, _bindings(shapes, "--shape", True), _bindings(dims, "--dim", False))


def _table_rows(value: Value, hops: int = 0) -> int | None:
    """Rows of the Gather table that ``value`` indexes, following reshapes and casts."""
    if hops > 8:
        return None
    for reader in value.users:
        if reader.op == "Gather" and reader.inputs[1] is value:
            table = reader.input(0).tensor_type
            return table.shape[int(reader.attrs.get("axis", 0)) % max(table.rank, 1)]
        if reader.op in ("Reshape", "Flatten", "Squeeze", "Unsqueeze", "Cast", "Identity"):
            found = _table_rows(reader.output, hops + 1)
            if found is not None:
                return found
    return None


def random_inputs(graph: Graph, seed: int = 0, int_high: int = 100) -> dict[str, np.ndarray]:
    """Seeded inputs: standard normal floats, booleans, integers in [0, int_high) — below the
    table size when the integers index a Gather."""
    rng = np.random.default_rng(seed)
    feeds = {}
    for v in graph.inputs:
        t = v.tensor_type
        dtype = numpy_dtype(t.dtype)
        if np.issubdtype(dtype, np.floating):
            feeds[v.name] = rng.standard_normal(t.shape).astype(dtype)
        elif dtype == np.bool_:
            feeds[v.name] = rng.integers(0, 2, t.shape).astype(np.bool_)
        else:
            rows = _table_rows(v)
            feeds[v.name] = rng.integers(0, min(int_high, rows) if rows else int_high, t.shape).astype(dtype)
    return feeds


def compile_command(args: argparse.Namespace) -> dict[str, Any]:
    from .codegen import compile_graph
    from .evaluate import evaluate_graph
    from .passes import optimize
    from .schedule import schedule

    graph = load_model(args.model, args.shape, args.dim)
    feeds = random_inputs(graph, args.seed, args.int_high)
    baseline = evaluate_graph(graph, feeds) if args.check else None
    optimize(graph, args.opt)
    schedule(graph)
    model = compile_graph(graph, cache_dir=args.cache_dir, backend=args.backend)
    try:
        outputs = model.run(feeds)
        report = model.report
        payload: dict[str, Any] = {
            "backend": model.backend,
            "pipeline": args.opt,
            "library": str(model.library_path),
            "kernels": dict(report.kernels) if report else {},
            "arena_mb": round(report.arena_bytes / 2**20, 2) if report else None,
            "weights_mb": round(report.weights_bytes / 2**20, 2) if report else None,
            "codegen_s": report.codegen_seconds if report else None,
            "build_s": report.build_seconds if report else None,
            "cached": report.cached if report else None,
            "outputs": {k: f"{v.dtype}{list(v.shape)}" for k, v in outputs.items()},
        }
        if baseline is not None:
            payload["max_abs_diff_vs_interpreter"] = max(
                (float(np.max(np.abs(outputs[k].astype(np.float64) - np.asarray(v, np.float64)), initial=0.0))
                 for k, v in baseline.items()), default=0.0)
        if args.bench:
            times = sorted(model.benchmark(feeds, warmup=2, repeat=args.bench))
            payload["latency_ms_median"] = round(1e3 * times[len(times) // 2], 4)
            payload["latency_ms_min"] = round(1e3 * times[0], 4)
        if args.output:
            payload["saved"] = str(model.save(args.output))
    finally:
        model.release()
    return payload


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(prog="mgc", description="Compile ONNX models for MI355X (hip backend).")
    parser.add_argument("--version", action="version", version=f"%(prog)s {__version__}")
    commands = parser.add_subparsers(dest="command", required=True)
    p = commands.add_parser("compile", help="optimize, build with the hip backend and run once")
    p.add_argument("model", help="ONNX file, or a bundled sample/config name")
    p.add_argument("--dim", action="append", default=[], metavar="NAME=N", help="a symbolic dimension (repeatable)")
    p.add_argument("--shape", action="append", default=[], metavar="INPUT=D0xD1",
                   help="a full static input shape (repeatable)")
    p.add_argument("--backend", default="hip", help="code generator (this build: hip)")
    p.add_argument("-O", "--opt", default="O3", help="O0..O3, an ablation level, or pass,pass,...")
    p.add_argument("-o", "--output", help="directory to save the library, weights and metadata")
    p.add_argument("--cache-dir", help="build cache (default ~/.cache/ml-graph-compiler)")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--int-high", type=int, default=100, help="upper bound for integer inputs")
    p.add_argument("--check", action="store_true", help="compare with the unoptimized graph evaluated on the CPU")
    p.add_argument("--bench", type=int, default=0, metavar="N", help="time N runs")
    p.add_argument("--json", action="store_true")
    return parser


def main(argv: Sequence[str] | None = None) -> int:
    args = build_parser().parse_args(argv)
    try:
        payload = compile_command(args)
    except CompilerError as exc:
        print(f"error: {exc}", file=sys.stderr)
        return 2
    if args.json:
        print(json.dumps(payload, indent=2))
    else:
        for key, value in payload.items():
            print(f"{key:>28}: {value}")
    return 0
