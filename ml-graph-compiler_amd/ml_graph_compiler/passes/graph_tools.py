"""Small graph queries and edits the rewrite passes share."""

from __future__ import annotations

from typing import Any

import numpy as np

from ..ir import Graph, Node, Value
from ..shape_inference import infer_node


def scalar_value(value: Value | None) -> float | None:
    """The number held by a one-element constant, else None."""
    if value is None or value.data is None or value.data.size != 1:
        return None
    return float(value.data.reshape(()))


def is_number(value: Value | None, target: float, rel: float = 1e-5) -> bool:
    """``value`` is a one-element constant within ``rel`` (relative, at least absolute) of
    ``target``."""
    got = scalar_value(value)
    return got is not None and abs(got - target) <= rel * max(1.0, abs(target))


def made_by(value: Value | None, *ops: str) -> Node | None:
    """The node that produced ``value`` when its operator is one of ``ops``."""
    node = None if value is None else value.producer
    return node if node is not None and node.op in ops else None


def sole_reader(graph: Graph, value: Value) -> Node | None:
    """The one node reading ``value``, provided it is read once and is not a graph output."""
    if len(value.users) != 1 or any(value is o for o in graph.outputs):
        return None
    return value.users[0]


def other_operand(node: Node, value: Value) -> Value | None:
    """The input of a binary node that is not ``value`` (the second when both are)."""
    return node.inputs[1] if node.inputs[0] is value else node.inputs[0]


def operand_with(node: Node | None, op: str, number: float) -> Value | None:
    """For ``node = op(v, number)`` (either order for Add and Mul) with ``v`` not a constant,
    return ``v``."""
    if node is None or node.op != op or len(node.inputs) != 2:
        return None
    orders = [(0, 1), (1, 0)] if op in ("Add", "Mul") else [(0, 1)]
    for keep, const in orders:
        kept = node.inputs[keep]
        if is_number(node.inputs[const], number) and kept is not None and not kept.is_constant:
            return kept
    return None


def in_use(graph: Graph, node: Node) -> bool:
    return any(o.users or any(o is g for g in graph.outputs) for o in node.outputs)


def place_before(graph: Graph, anchor: Node, op: str, inputs: list[Value | None],
                 attrs: dict[str, Any] | None = None, n_outputs: int = 1) -> Node:
    """A new node placed right before ``anchor``, its output types inferred."""
    node = graph.add_node(op, inputs, n_outputs=n_outputs, attrs=attrs, index=graph.nodes.index(anchor))
    infer_node(node)
    return node


def substitute(graph: Graph, old: Node, op: str, inputs: list[Value | None], attrs: dict[str, Any] | None = None,
               anchor: Node | None = None) -> Node:
    """Compute ``old``'s first output with a new node (placed before ``anchor``, default ``old``)
    and point every reader at it; ``old`` becomes dead."""
    new = place_before(graph, anchor or old, op, inputs, attrs)
    graph.replace_all_uses(old.outputs[0], new.output)
    return new


def per_channel(value: Value | None, n: int, axis_from_end: int) -> np.ndarray | None:
    """A constant usable as a length-``n`` vector along axis ``-axis_from_end``: a scalar
    (broadcast), or exactly n elements lying on that axis. Returned flat, float32."""
    if value is None or value.data is None:
        return None
    data = value.data
    if data.size == 1:
        return np.full(n, float(data.reshape(())), dtype=np.float32)
    on_axis = data.ndim >= axis_from_end and data.shape[data.ndim - axis_from_end] == n
    return data.reshape(n).astype(np.float32) if data.size == n and on_axis else None
