"""Test helpers: one-operator IR graphs and comparison of the hip backend with the oracle.

``op_graph`` is the IR counterpart of the reference's ``op_model`` (tests/helpers.py:23-59):
inputs listed in ``const`` become constants, the others graph inputs fed from the arrays.
"""

from __future__ import annotations

from pathlib import Path
from typing import Any

import numpy as np

from ml_graph_compiler.ir import Graph, TensorType, dtype_name
from ml_graph_compiler.passes import optimize
from ml_graph_compiler.schedule import schedule
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle

rng = np.random.default_rng(1)


def f32(*shape: int) -> np.ndarray:
    return np.asarray(rng.standard_normal(shape), dtype=np.float32)


def pos(*shape: int) -> np.ndarray:
    return np.asarray(rng.random(shape) + 0.5, dtype=np.float32)


def op_graph(
    op: str,
    inputs: list[np.ndarray | None],
    const: set[int] | None = None,
    attrs: dict[str, Any] | None = None,
    n_outputs: int = 1,
) -> tuple[Graph, dict[str, np.ndarray]]:
    const = const or set()
    g = Graph("single")
    values, feeds = [], {}
    for i, array in enumerate(inputs):
        if array is None:
            values.append(None)
            continue
        a = np.asarray(array)
        if i in const:
            values.append(g.constant(a, f"in{i}"))
        else:
            values.append(g.add_input(f"in{i}", TensorType(dtype_name(a.dtype), tuple(a.shape))))
            feeds[f"in{i}"] = a
    node = g.add_node(op, values, n_outputs, attrs or {}, name="node", output_names=[f"out{i}" for i in range(n_outputs)])
    for i, out in enumerate(node.outputs):
        g.add_output(out, f"out{i}")
    infer_shapes(g)
    return g, feeds


def compile_hip(graph: Graph, cache: Path, opt: str = "O3", **kwargs: Any):
    from ml_graph_compiler.codegen import compile_graph

    optimize(graph, opt)
    schedule(graph)
    return compile_graph(graph, cache_dir=cache, **kwargs)


def check_hip(
    graph: Graph,
    feeds: dict[str, np.ndarray],
    cache: Path,
    opt: str = "O0",
    rtol: float = 1e-4,
    atol: float = 1e-5,
    exact: bool = False,
) -> dict[str, np.ndarray]:
    """Compile ``graph`` with the hip backend at ``opt``, run it and compare every output with
    the oracle run on the unoptimized graph; returns the hip outputs. Integer and bool outputs
    always compare bit for bit; ``exact`` makes float outputs do so too (pure data movement:
    Gather, Transpose, Slice, ...)."""
    expected = oracle.run_graph(graph, feeds)
    model = compile_hip(graph, cache, opt)
    try:
        got = model.run(feeds)
    finally:
        model.release()
    assert set(got) == set(expected)
    for name, value in expected.items():
        assert got[name].shape == value.shape, (name, got[name].shape, value.shape)
        assert got[name].dtype == value.dtype, (name, got[name].dtype, value.dtype)
        if np.issubdtype(value.dtype, np.floating) and not exact:
            np.testing.assert_allclose(got[name], value, rtol=rtol, atol=atol, err_msg=name)
        else:
            np.testing.assert_array_equal(got[name], value, err_msg=name)
    return got


def named_graph(
    nodes: list[tuple[str, list[str], list[str], dict[str, Any]]],
    inputs: list[tuple[str, tuple[int, ...], str]],
    outputs: list[str],
    inits: list[tuple[str, np.ndarray]] = (),
) -> Graph:
    """A graph from name-wired nodes, like the reference tests' onnx.helper models: inputs are
    (name, shape, dtype), inits become constants, an empty input name is an omitted input."""
    g = Graph("t")
    env: dict[str, Any] = {}
    for name, array in inits:
        env[name] = g.constant(np.asarray(array), name)
    for name, shape, dtype in inputs:
        env[name] = g.add_input(name, TensorType(dtype, tuple(shape)))
    for op, ins, outs, attrs in nodes:
        node = g.add_node(op, [env[n] if n else None for n in ins], len(outs), attrs, output_names=outs)
        for n, v in zip(outs, node.outputs):
            env[n] = v
    for name in outputs:
        g.add_output(env[name], name)
    infer_shapes(g)
    return g


def same_numerics(make, passes: str, rtol: float = 1e-5, atol: float = 1e-5) -> Graph:
    """Optimize a fresh graph from ``make()`` with ``passes`` and check the oracle agrees with
    the unoptimized graph on seeded inputs; returns the optimized graph."""
    from ml_graph_compiler.passes import optimize

    reference = make()
    feeds = oracle.random_feeds(reference, 3, int_high=20)
    expected = oracle.run_graph(reference, feeds)
    graph = make()
    optimize(graph, passes)
    got = oracle.run_graph(graph, feeds)
    for name, value in expected.items():
        assert got[name].shape == value.shape
        np.testing.assert_allclose(got[name], value, rtol=rtol, atol=atol, err_msg=name)
    return graph


def batch_norm_statistics(graph: Graph, feeds: dict[str, np.ndarray]) -> list[tuple[np.ndarray, np.ndarray]]:
    """Calibrate the running statistics of every BatchNormalization of ``graph`` on ``feeds``:
    run the oracle node by node and, at each BatchNormalization, replace its mean and variance
    with the batch mean and (biased) variance of its input over every axis but the channel axis
    before evaluating it, so its output has the drawn scale and shift per channel and the
    network's activations stay O(1) at any depth. Returns the (mean, var) pairs in node order;
    ``graph`` is left calibrated."""
    env = dict((id(v), a) for v, a in zip(graph.inputs, (oracle.check_feeds(graph, feeds)[v.name] for v in graph.inputs)))
    stats = []

    def get(v):
        return None if v is None else (v.data if v.data is not None else env[id(v)])

    for node in graph.nodes:
        if node.op == "BatchNormalization":
            x = get(node.input(0)).astype(np.float64)
            axes = (0,) + tuple(range(2, x.ndim))
            node.input(3).data = x.mean(axis=axes).astype(np.float32)
            node.input(4).data = x.var(axis=axes).astype(np.float32)
            stats.append((node.input(3).data, node.input(4).data))
        for v, a in zip(node.outputs, oracle.run_node(node, [get(v) for v in node.inputs])):
            env[id(v)] = a
    return stats


def with_batch_norm_statistics(graph: Graph, stats: list[tuple[np.ndarray, np.ndarray]]) -> Graph:
    """``graph`` with the BatchNormalization statistics ``stats`` (from batch_norm_statistics on
    a graph of the same builder and seed, any batch) set in node order."""
    bns = [n for n in graph.nodes if n.op == "BatchNormalization"]
    assert len(bns) == len(stats)
    for node, (mean, var) in zip(bns, stats):
        assert node.input(3).data.shape == mean.shape
        node.input(3).data, node.input(4).data = mean, var
    return graph
