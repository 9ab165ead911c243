"""Helpers shared by the passes (reference: src/ml_graph_compiler/passes/util.py:1-84)."""

from __future__ import annotations

from typing import Any

import numpy as np

from ..ir import Graph, Node, Value
from ..shape_inference import infer_node


def const(value: Value | None) -> np.ndarray | None:
    return None if value is None else value.data


def scalar(value: Value | None) -> float | None:
    """The value of a one-element constant, else None."""
    data = const(value)
    if data is None or data.size != 1:
        return None
    return float(data.reshape(()))


def is_scalar(value: Value | None, target: float, rel: float = 1e-5) -> bool:
    s = scalar(value)
    return s is not None and abs(s - target) <= rel * max(1.0, abs(target))


def producer(value: Value | None, op: str | tuple[str, ...]) -> Node | None:
    """The node producing ``value`` when its operator is ``op`` (or one of ``op``)."""
    if value is None or value.producer is None:
        return None
    wanted = (op,) if isinstance(op, str) else op
    return value.producer if value.producer.op in wanted else None


def only_user(value: Value, graph: Graph) -> Node | None:
    """The single consumer of a value that is not a graph output."""
    if len(value.users) != 1 or value in graph.outputs:
        return None
    return value.users[0]


def binary_with_const(node: Node | None, op: str, target: float) -> Value | None:
    """x when ``node`` is op(x, c) (or op(c, x) for Add/Mul) with scalar constant c == target."""
    if node is None or node.op != op or len(node.inputs) != 2:
        return None
    a, b = node.inputs
    if is_scalar(b, target) and a is not None and not a.is_constant:
        return a
    if op in ("Add", "Mul") and is_scalar(a, target) and b is not None and not b.is_constant:
        return b
    return None


def insert_node(
    graph: Graph,
    op: str,
    inputs: list[Value | None],
    before: Node,
    attrs: dict[str, Any] | None = None,
    n_outputs: int = 1,
    name: str = "",
) -> Node:
    """Insert a typed node immediately before ``before``."""
    node = graph.add_node(
        op, inputs, n_outputs=n_outputs, attrs=attrs, name=name, index=graph.nodes.index(before)
    )
    infer_node(node)
    return node


def remove_dead(graph: Graph, nodes: list[Node]) -> int:
    """Remove the listed nodes (last first) whose outputs are no longer used."""
    count = 0
    for node in reversed(nodes):
        if node in graph.nodes and not any(o.users or o in graph.outputs for o in node.outputs):
            graph.remove_node(node)
            count += 1
    return count
